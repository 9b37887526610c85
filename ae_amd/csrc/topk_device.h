// Device building blocks of the top-k softmax gating and of the one-wave routing, shared by the
// routing kernels (routing.hip) and the expert kernels that route small batches themselves
// (experts.hip).
#pragma once

#include "smx_kernels.h"

namespace smx {

// ---------------------------------------------------------------------------------------
// Top-k softmax, G lanes per token (G = 8, 16, 32 or 64; a wave holds 64/G tokens). Lane j of
// a group holds experts j + G*i, i < PL (PL = 4 only for G = 64: up to 256 experts). On
// return lane j < k of each group holds the j-th pick (descending probability, ties to the
// lower expert index). The arithmetic (max, exp_nonpos, per-lane sequential sum, butterfly
// over the group with offsets 1, 2, ..., G/2, p = ex * (1/sum), renormalisation by division
// with the sum taken in j order) equals the oracle's 64-lane butterfly bit for bit: with
// E <= G every lane at or past G holds an exact zero, so the oracle's steps at offsets >= G
// only add zeros.
// Semantics follow select_experts as called at specmoe/layers/FusedMoE.py:174-185.
//
// NB wave-passes (NB groups of tokens) are computed in lockstep: every butterfly step is
// issued for all NB before the next, so the NB independent shuffle chains hide each
// other's latency.
// ---------------------------------------------------------------------------------------
template <int G, int PL>
struct TopkGroup {
  static_assert(PL == 1 || G == kWave, "several experts per lane only with whole-wave groups");
  static constexpr int kTokens = kWave / G;  // tokens per wave-pass
};

// Lane j of a group reads experts j + G*i of token t. Experts past E read -inf (never
// selected); a token past T reads zeros so that its arithmetic stays finite (its results
// are discarded).
// Every lane loads (from a clamped, in-bounds index; T >= 1) and then selects, so that the loads
// of several passes are all in flight before the first is waited for (a load under a branch is
// waited for inside the branch).
template <int LDT, int G, int PL>
__device__ __forceinline__ void load_logits(const void* logits, int t, int T, int E, float (&v)[PL]) {
  const int j = lane_id() % G;
  const int64_t row = static_cast<int64_t>(t < T ? t : T - 1) * E;
#pragma unroll
  for (int i = 0; i < PL; ++i) {
    const int e = j + G * i;
    const float x = load_as_f32<LDT>(logits, row + (e < E ? e : E - 1));
    v[i] = e >= E ? -__builtin_inff() : (t < T ? x : 0.0f);
  }
}

// Cross-lane exchange within rows of 16 lanes by DPP (a VALU operand modifier, no LDS
// round trip). Controls: quad_perm [1,0,3,2] (lane ^ 1), quad_perm [2,3,0,1] (lane ^ 2),
// row_half_mirror (lane i <-> 7 - i within 8), row_mirror (lane i <-> 15 - i within 16).
constexpr int kDppXor1 = 0xB1;
constexpr int kDppXor2 = 0x4E;
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ float readlane(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// op-reduction over the G lanes of each group; every lane of the group gets the result.
// The steps pair lane i with i^1, i^2, then (on values already equal across each quad,
// resp. half-row) with the mirrored lane, which holds the same value as lane i^4 (resp.
// i^8); rows are combined as op(op(r0, r1), op(r2, r3)) from lanes 0, 16, 32, 48. For a
// commutative op every intermediate value equals that of the xor butterfly over offsets
// 1, 2, 4, ..., G/2 (for fp32 addition bit for bit: a + b == b + a exactly).
template <int G, typename Op>
__device__ __forceinline__ float group_reduce(float v, Op op) {
  v = op(v, dpp<kDppXor1>(v));
  v = op(v, dpp<kDppXor2>(v));
  v = op(v, dpp<kDppHalfMirror>(v));
  if constexpr (G >= 16) v = op(v, dpp<kDppMirror>(v));
  if constexpr (G >= 32) {
    const float r0 = readlane(v, 0), r1 = readlane(v, 16), r2 = readlane(v, 32), r3 = readlane(v, 48);
    if constexpr (G == 32) v = lane_id() < 32 ? op(r0, r1) : op(r2, r3);
    else v = op(op(r0, r1), op(r2, r3));
  }
  return v;
}

// (p, e) pair order: larger p first, ties to the lower expert index.
__device__ __forceinline__ bool better(float op, int oe, float bp, int be) {
  return op > bp || (op == bp && oe < be);
}

template <int CTRL>
__device__ __forceinline__ void argmax_step(float& bp, int& be) {
  const float op = dpp<CTRL>(bp);
  const int oe = dpp<CTRL>(be);
  if (better(op, oe, bp, be)) { bp = op; be = oe; }
}

// Arg-max over the G lanes of each group, the same reduction shape as group_reduce.
template <int G>
__device__ __forceinline__ void group_argmax(float& bp, int& be) {
  argmax_step<kDppXor1>(bp, be);
  argmax_step<kDppXor2>(bp, be);
  argmax_step<kDppHalfMirror>(bp, be);
  if constexpr (G >= 16) argmax_step<kDppMirror>(bp, be);
  if constexpr (G >= 32) {
    float p[4];
    int e[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p[r] = readlane(bp, 16 * r);
      e[r] = __builtin_amdgcn_readlane(be, 16 * r);
    }
    if (better(p[1], e[1], p[0], e[0])) { p[0] = p[1]; e[0] = e[1]; }
    if (better(p[3], e[3], p[2], e[2])) { p[2] = p[3]; e[2] = e[3]; }
    if constexpr (G == 32) {
      const bool hi = lane_id() >= 32;
      bp = hi ? p[2] : p[0];
      be = hi ? e[2] : e[0];
    } else {
      if (better(p[2], e[2], p[0], e[0])) { p[0] = p[2]; e[0] = e[2]; }
      bp = p[0];
      be = e[0];
    }
  }
}

template <int G, int PL, int NB>
__device__ __forceinline__ void group_topk_softmax(float (&p)[NB][PL], int E, int k, bool renorm,
                                                   float (&w_out)[NB], int (&id_out)[NB]) {
#pragma clang fp contract(off)
  const int lane = lane_id();
  const int j = lane % G;
  const int base = lane - j;
  float m[NB], s[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    m[b] = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < PL; ++i) m[b] = fmaxf(m[b], p[b][i]);
    m[b] = group_reduce<G>(m[b], [](float a, float c) { return fmaxf(a, c); });
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) {
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      const int e = j + G * i;
      p[b][i] = (e < E) ? exp_nonpos(p[b][i] - m[b]) : 0.0f;
      s[b] = (i == 0) ? p[b][i] : s[b] + p[b][i];
    }
    s[b] = group_reduce<G>(s[b], [](float a, float c) { return a + c; });
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const float inv = 1.0f / s[b];
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      const int e = j + G * i;
      p[b][i] = (e < E) ? p[b][i] * inv : -1.0f;  // -1 marks "not selectable"
    }
    w_out[b] = 0.0f;
    id_out[b] = -1;
  }
  for (int jj = 0; jj < k; ++jj) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      float bp = -2.0f;
      int be = 0x7fffffff;
#pragma unroll
      for (int i = 0; i < PL; ++i)
        if (p[b][i] > bp) { bp = p[b][i]; be = j + G * i; }  // ascending e: strict > keeps lowest
      group_argmax<G>(bp, be);
      if (j == be % G) {
#pragma unroll
        for (int i = 0; i < PL; ++i)
          if (i == be / G) p[b][i] = -1.0f;
      }
      if (j == jj) { w_out[b] = bp; id_out[b] = be; }
    }
  }
  if (renorm) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      float sum = 0.0f;
      for (int jj = 0; jj < k; ++jj) {
        const float v = (G == kWave) ? readlane(w_out[b], jj) : __shfl(w_out[b], base + jj, kWave);
        sum = (jj == 0) ? v : sum + v;
      }
      if (j < k) w_out[b] = w_out[b] / sum;
    }
  }
}

// Top-k for one expert per lane (E <= G <= 64): the softmax as above, then k selection rounds,
// each a group max of p (DPP steps) and the lowest lane of the group holding that max (one
// ballot). Equal p are equal bits (p >= +0, no NaN), so the lowest lane among them is the
// lower expert index: descending p, ties to the lower index, as select_experts orders them.
// Lane j picked in round r gets slot_out = r (else -1). Renormalisation divides by the picks'
// sum taken in pick order. Against a ranking by 64-bit keys compared from LDS (each lane
// counting the larger keys of its group, ~1 us per token pass at E = 64: the LDS reads
// issue two at a time), the rounds are a few dozen dependent VALU steps each.
template <int G>
__device__ __forceinline__ void group_topk_select(float& p, int E, int k, bool renorm, float& w_out,
                                                  int& id_out, int& slot_out) {
#pragma clang fp contract(off)
  const int lane = lane_id();
  const int j = lane % G;
  const int base = lane - j;
  const bool valid = j < E;
  const float m = group_reduce<G>(p, [](float a, float c) { return fmaxf(a, c); });
  const float ex = valid ? exp_nonpos(p - m) : 0.0f;
  const float s = group_reduce<G>(ex, [](float a, float c) { return a + c; });
  const float pr = ex * (1.0f / s);
  // below every probability: never the max while k <= E (a NaN probability, from NaN logits,
  // ranks there too, so every round still picks one lane)
  float q = (valid && pr == pr) ? pr : -1.0f;
  int slot = -1;
  float sum = 0.0f;
  for (int r = 0; r < k; ++r) {
    const float mx = group_reduce<G>(q, [](float a, float c) { return fmaxf(a, c); });
    const uint64_t eq = ballot(q == mx);
    const uint64_t gm = G == kWave ? eq : (eq >> base) & ((uint64_t{1} << G) - 1);
    const int pick = __builtin_ctzll(gm);
    if (j == pick) {
      slot = r;
      q = -2.0f;
    }
    sum = (r == 0) ? mx : sum + mx;
  }
  slot_out = slot;
  id_out = j;
  w_out = renorm ? pr / sum : pr;
}

// The tokens of kTokBatch consecutive wave-passes: token t = first + b * stride for this
// lane's group. All logit loads are issued before any token is computed, so a wave pays one
// load latency per batch. fn(t, w, id) is called on every lane (t may be >= T).
// fn(t, slot, w, id) is called for every pick of token t (t < T): slot in [0, k).
template <int LDT, int G, int PL, typename Fn>
__device__ __forceinline__ void topk_batch(const void* logits, int T, int E, int k, bool renorm,
                                           int first, int stride, Fn&& fn) {
  float v[kTokBatch][PL];
#pragma unroll
  for (int b = 0; b < kTokBatch; ++b) load_logits<LDT, G, PL>(logits, first + b * stride, T, E, v[b]);
  float w[kTokBatch];
  int id[kTokBatch];
  int slot[kTokBatch];
  if constexpr (PL == 1) {
#pragma unroll
    for (int b = 0; b < kTokBatch; ++b) group_topk_select<G>(v[b][0], E, k, renorm, w[b], id[b], slot[b]);
  } else {
    group_topk_softmax<G, PL, kTokBatch>(v, E, k, renorm, w, id);
    const int j = lane_id() % G;
#pragma unroll
    for (int b = 0; b < kTokBatch; ++b) slot[b] = j < k ? j : -1;
  }
#pragma unroll
  for (int b = 0; b < kTokBatch; ++b) {
    const int t = first + b * stride;
    if (t < T && slot[b] >= 0) fn(t, slot[b], w[b], id[b]);
  }
}

// ---------------------------------------------------------------------------------------
// Top-k softmax over blocks of consecutive experts (E <= 64): lane j of a group of G lanes
// (G = 1, 2, 4 or 8, 8G >= E) holds experts 8j .. 8j+7 of its token, so a wave computes 64/G
// tokens per pass and most of the work is lane-local. The softmax sum adds the lane's eight
// values pairwise, ((x0+x1)+(x2+x3))+((x4+x5)+(x6+x7)), then over the group's lanes by the
// butterfly with offsets 1, 2, 4: the same binary tree as the 64-lane butterfly of
// group_topk_select (expert e on lane e, offsets 1..32), whose levels past 8G add exact
// zeros, so probabilities, picks and weights equal group_topk_select's bit for bit. Each
// selection round takes the lane's best value (strict > over ascending experts keeps the
// lower index) and an arg-max over the group (ties to the lower index); NaN probabilities
// rank at -1 and picked experts at -2, as in group_topk_select.
// ---------------------------------------------------------------------------------------
// Lanes per token of the block form: the fewest (a power of two) whose blocks cover E <= 64.
__host__ __device__ constexpr int block_group_for(int E) {
  return E <= 8 ? 1 : E <= 16 ? 2 : E <= 32 ? 4 : 8;
}

template <int G, typename Op>
__device__ __forceinline__ float lane_group_reduce(float v, Op op) {
  if constexpr (G >= 2) v = op(v, dpp<kDppXor1>(v));
  if constexpr (G >= 4) v = op(v, dpp<kDppXor2>(v));
  if constexpr (G >= 8) v = op(v, dpp<kDppHalfMirror>(v));
  return v;
}

template <int G>
__device__ __forceinline__ void lane_group_argmax(float& bp, int& be) {
  if constexpr (G >= 2) argmax_step<kDppXor1>(bp, be);
  if constexpr (G >= 4) argmax_step<kDppXor2>(bp, be);
  if constexpr (G >= 8) argmax_step<kDppHalfMirror>(bp, be);
}

// Experts 8j .. 8j+7 of token t (clamped, in-bounds loads; experts past E read -inf, a token
// past T reads zeros).
template <int LDT, int G>
__device__ __forceinline__ void load_logit_block(const void* logits, int t, int T, int E,
                                                 float (&v)[kBlockExperts]) {
  const int j = lane_id() % G;
  const int64_t row = static_cast<int64_t>(t < T ? t : T - 1) * E;
#pragma unroll
  for (int i = 0; i < kBlockExperts; ++i) {
    const int e = kBlockExperts * j + i;
    const float x = load_as_f32<LDT>(logits, row + (e < E ? e : E - 1));
    v[i] = e >= E ? -__builtin_inff() : (t < T ? x : 0.0f);
  }
}

// The k picks of the lane's token, in pick order; lane j keeps picks j, j + G, ... in
// w_out[r / G], id_out[r / G] (pick r), renormalised when asked.
template <int G>
__device__ __forceinline__ void block_topk_select(float (&v)[kBlockExperts], int E, int k, bool renorm,
                                                  float (&w_out)[(kMaxTopK + G - 1) / G],
                                                  int (&id_out)[(kMaxTopK + G - 1) / G]) {
#pragma clang fp contract(off)
  const int j = lane_id() % G;
#pragma unroll
  for (int s2 = 0; s2 < (kMaxTopK + G - 1) / G; ++s2) {
    w_out[s2] = 0.0f;
    id_out[s2] = -1;
  }
  float m = v[0];
#pragma unroll
  for (int i = 1; i < kBlockExperts; ++i) m = fmaxf(m, v[i]);
  m = lane_group_reduce<G>(m, [](float a, float c) { return fmaxf(a, c); });
  float ex[kBlockExperts];
#pragma unroll
  for (int i = 0; i < kBlockExperts; ++i)
    ex[i] = kBlockExperts * j + i < E ? exp_nonpos(v[i] - m) : 0.0f;
  float s = ((ex[0] + ex[1]) + (ex[2] + ex[3])) + ((ex[4] + ex[5]) + (ex[6] + ex[7]));
  s = lane_group_reduce<G>(s, [](float a, float c) { return a + c; });
  const float inv = 1.0f / s;
  float q[kBlockExperts];
#pragma unroll
  for (int i = 0; i < kBlockExperts; ++i) {
    const float pr = ex[i] * inv;
    q[i] = (kBlockExperts * j + i < E && pr == pr) ? pr : -1.0f;
  }
  float sum = 0.0f;
#pragma unroll
  for (int r = 0; r < kMaxTopK; ++r) {
    if (r >= k) break;
    float bp = q[0];
    int bi = 0;
#pragma unroll
    for (int i = 1; i < kBlockExperts; ++i)
      if (q[i] > bp) { bp = q[i]; bi = i; }
    int be = kBlockExperts * j + bi;
    lane_group_argmax<G>(bp, be);
    if (be / kBlockExperts == j) {
#pragma unroll
      for (int i = 0; i < kBlockExperts; ++i)
        if (i == be % kBlockExperts) q[i] = -2.0f;
    }
    if (j == r % G) {
      // the pick's probability: its rank value, or NaN where it ranked as -1
      w_out[r / G] = bp >= 0.0f ? bp : __builtin_nanf("");
      id_out[r / G] = be;
    }
    sum = (r == 0) ? bp : sum + bp;
  }
  if (renorm) {
#pragma unroll
    for (int s2 = 0; s2 < (kMaxTopK + G - 1) / G; ++s2) w_out[s2] = w_out[s2] / sum;
  }
}

// NB consecutive passes of 64/G tokens (token t = first + b * stride for this lane's group):
// every logit load is issued before any token is computed. fn(t, slot, w, id) is called for
// every pick of token t < T.
template <int LDT, int G, int NB, typename Fn>
__device__ __forceinline__ void topk_block_batch(const void* logits, int T, int E, int k, bool renorm,
                                                 int first, int stride, Fn&& fn) {
  constexpr int kPer = (kMaxTopK + G - 1) / G;
  float v[NB][kBlockExperts];
#pragma unroll
  for (int b = 0; b < NB; ++b) load_logit_block<LDT, G>(logits, first + b * stride, T, E, v[b]);
  const int j = lane_id() % G;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    float w[kPer];
    int id[kPer];
    block_topk_select<G>(v[b], E, k, renorm, w, id);
    const int t = first + b * stride;
    if (t < T) {
#pragma unroll
      for (int s = 0; s < kPer; ++s)
        if (j + G * s < k) fn(t, j + G * s, w[s], id[s]);
    }
  }
}

struct AlignOutputs {
  // compact lists for the expert kernels (may be null)
  int32_t* hdr;         // [0] = number of work ranges, [1] = dropped-assignment flag
  RangeRec* ranges;     // [active experts + N / span]
  int span;             // sorted positions per range
  int32_t* sorted_f;    // [N]
  int32_t* tmask;       // [T] per token: bit j set if assignment t*k+j is routable
  int32_t* fpos;        // [N] sorted position of each routable assignment
  int64_t* fslot;       // [N] pool slot of each routable assignment (route only)
  bool by_expert;       // ranges[e] = expert e's record for every e < E (cnt 0 when it has no
                        // routable assignment) instead of the compact list (second output only)
  // reference-format outputs (may be null)
  int32_t* sorted_ids;  // [N + E*(BM-1)]
  int32_t* expert_ids;  // [ceil((N + E*(BM-1)) / BM)]
  int32_t* ntp;         // [1]
  int bm;
};

// Lanes of the wave whose (valid) expert id equals this lane's: one ballot per id bit.
__device__ __forceinline__ uint64_t same_expert_lanes(int e, bool valid, int nbits) {
  uint64_t same = ballot(valid);
  for (int b = 0; b < nbits; ++b) {
    const bool bit = (e >> b) & 1;
    const uint64_t m = ballot(bit);
    same &= bit ? m : ~m;
  }
  return same;
}

// ---------------------------------------------------------------------------------------
// The expert sort by one wave, for at most kSortWaveMax assignments over at most 64 experts
// (lane e owns expert e): chunks of 64 assignments in order, the lanes of a chunk with the
// same expert found with one ballot per id bit, counts per expert in LDS, one wave scan over
// the experts, then the scatter. No workgroup barriers (a wave's LDS accesses execute in
// program order). Stable: within an expert, assignments appear in ascending f. Inputs:
// ids[f] (-1 dropped, -2 out of range: dropped and flagged), slot[e] (kCheckSlots: < 0 drops
// the expert's assignments and flags them). Every non-null member of `out` and of `out2` is
// written (out2: a second copy of the records, e.g. in a workgroup's LDS). The records are
// those of the multi-wave sort (align_block in routing.hip), element for element.
// Measured against the multi-wave sort (us per layer): DeepSeek-V2-Lite 8 tokens (48
// assignments, fused top-k) 124.1 -> 122.2, 32 tokens (192) 181.1 -> 180.2; Mixtral 64
// tokens (128) 438.1 -> 436.5; Qwen1.5-MoE 64 tokens (256) 190.3 -> 189.7; DeepSeek-V2-Lite
// 64 tokens (384) 198.4 -> 199.3, so the limit is 256.
// ---------------------------------------------------------------------------------------

struct SortWaveLds {
  int cnt[kWave + 1];
  int off[kWave + 1];
  int seg[kWave + 1];
  int run[kWave];
};

// Inlined: as a call it holds its output structs in scratch, and the call waits for every
// vector load in flight (the gate/up launch issues its first weight chunks before routing).
template <bool kCheckSlots>
__device__ __forceinline__ void sort_wave(const int16_t* ids, const int64_t* slot, int N, int E, SortWaveLds& sc,
                          const AlignOutputs& out, const AlignOutputs& out2) {
  const int lane = lane_id();
  const int nbits = E > 1 ? 32 - __clz(E - 1) : 0;
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
  const int nch = (N + kWave - 1) / kWave;
  int* run = sc.run;  // per expert: count, then running sorted position
  run[lane] = 0;
  bool bad = false;
  __builtin_amdgcn_wave_barrier();
  for (int c = 0; c < nch; ++c) {
    const int f = c * kWave + lane;
    int e = f < N ? static_cast<int>(ids[f]) : -1;
    if (e == -2 || (kCheckSlots && e >= 0 && slot[e] < 0)) {
      bad = true;
      e = -1;
    }
    const uint64_t same = same_expert_lanes(e, e >= 0, nbits);
    if (e >= 0 && (same & below) == 0) run[e] += __popcll(same);
    __builtin_amdgcn_wave_barrier();
  }
  // exclusive scans over the experts: compact offset, block-padded segment, active count, range
  const int ce = lane < E ? run[lane] : 0;
  const int bm = out.bm > 0 ? out.bm : 1;
  const int span = out.span > 0 ? out.span : 1;
  const int pad = div_small(ce + bm - 1, bm, 1.0f / bm) * bm;
  const int act = ce > 0 ? 1 : 0;
  const int nr = div_small(ce + span - 1, span, 1.0f / span);
  const int ic = wave_incl_scan(ce), ip = wave_incl_scan(pad), ia = wave_incl_scan(act),
            ir = wave_incl_scan(nr);
  const int off = ic - ce, seg = ip - pad, br = ir - nr;
  const int seg_total = last_lane(ip);
  const int ranges_total = last_lane(ir);
  const int active_total = last_lane(ia);
  const bool any_bad = ballot(bad) != 0;
  if (lane < E) {
    sc.cnt[lane] = ce;
    sc.off[lane] = off;
    sc.seg[lane] = seg;
    run[lane] = off;
    RangeRec rec{};
    rec.slot = kCheckSlots ? slot[lane] : -1;
    rec.off = off;
    rec.cnt = ce;
    rec.key = lane;
    rec.j0 = br;
    rec.nr = nr;
    if (ce > 0 && (out.ranges || (out2.ranges && !out2.by_expert))) {
      for (int r = 0; r < nr; ++r) {
        if (out.ranges) out.ranges[br + r] = rec;
        if (out2.ranges && !out2.by_expert) out2.ranges[br + r] = rec;
      }
    }
    if (out2.ranges && out2.by_expert) out2.ranges[lane] = rec;  // every expert, cnt 0 if idle
  }
  if (lane == 0) {
    sc.seg[E] = seg_total;
    if (out.hdr) {
      out.hdr[0] = ranges_total;
      out.hdr[1] = any_bad ? 1 : 0;
      out.hdr[kHdrSingleRanges] = ranges_total == active_total ? 1 : 0;
    }
    if (out2.hdr) {
      out2.hdr[0] = ranges_total;
      out2.hdr[1] = any_bad ? 1 : 0;
      out2.hdr[kHdrSingleRanges] = ranges_total == active_total ? 1 : 0;
    }
    if (out.ntp) out.ntp[0] = seg_total;
  }
  __builtin_amdgcn_wave_barrier();
  // scatter: every lane reads its expert's running position before the rank-0 lane advances it
  for (int c = 0; c < nch; ++c) {
    const int f = c * kWave + lane;
    int e = f < N ? static_cast<int>(ids[f]) : -1;
    if (e == -2 || (kCheckSlots && e >= 0 && slot[e] < 0)) e = -1;
    const uint64_t same = same_expert_lanes(e, e >= 0, nbits);
    if (e >= 0) {
      const int rank = __popcll(same & below);
      const int pos = run[e] + rank;
      if (out.sorted_f) out.sorted_f[pos] = f;
      if (out2.sorted_f) out2.sorted_f[pos] = f;
      if (out.fpos) {
        out.fpos[f] = pos;
        out.fslot[f] = kCheckSlots ? slot[e] : -1;
      }
      if (out.sorted_ids) out.sorted_ids[sc.seg[e] + (pos - sc.off[e])] = f;
      if (rank == 0) run[e] = pos + __popcll(same);
    }
    __builtin_amdgcn_wave_barrier();
  }
  // reference format: sentinel padding and per-block expert ids
  if (out.sorted_ids) {
    const int len = N + E * (bm - 1);
    const int nblocks = (len + bm - 1) / bm;
    for (int e = 0; e < E; ++e) {
      for (int p = sc.seg[e] + sc.cnt[e] + lane; p < sc.seg[e + 1]; p += kWave) out.sorted_ids[p] = N;
      for (int b = sc.seg[e] / bm + lane; b < sc.seg[e + 1] / bm; b += kWave) out.expert_ids[b] = e;
    }
    for (int p = seg_total + lane; p < len; p += kWave) out.sorted_ids[p] = N;
    for (int b = seg_total / bm + lane; b < nblocks; b += kWave) out.expert_ids[b] = -1;
  }
}

// ---------------------------------------------------------------------------------------
// Routing of a small batch (T*k <= 64 assignments, E <= 64) by one wave, without workgroup
// barriers: the top-k of every token (all logits loaded up front, one latency), then lane f
// takes assignment f and the sort is done with ballots. For each lane the lanes with the same
// expert and the lanes with a smaller expert are found bit by bit from the top id bit down
// (eq: lanes agreeing on the bits so far; a lane whose id has a 1 where an eq lane has a 0
// ranks that lane below it); the sorted position is (#smaller) + (#same below this lane), so
// within an expert assignments stay in ascending f, and the active-expert index is the number
// of smaller experts present. The records are those of the multi-wave routing kernel (same
// order, same values). With logits null the ids come from ids_in (out-of-range ids dropped).
// ---------------------------------------------------------------------------------------

// Outputs of the one-wave routing; null members are not written.
struct SmallRouteOut {
  float* w = nullptr;           // [T*k] top-k weights
  int32_t* ids = nullptr;       // [T*k] top-k expert ids
  int32_t* hdr = nullptr;       // [0] work ranges, [1] dropped flag
  RangeRec* ranges = nullptr;   // [kSmallRangesMax] ceil(cnt / span) per active expert
  int32_t* sorted_f = nullptr;  // [T*k]
  int32_t* tmask = nullptr;     // [T]
  int32_t* fpos = nullptr;      // [T*k]
  int64_t* fslot = nullptr;     // [T*k]
};

struct SmallRouteLds {
  int ids[kWave];
  int64_t slot[kWave];
  int nr[kWave];  // ranges per active expert, then the first range of each (several-range case)
};


// Called by one whole wave; writes every non-null member of `a` and of `b`. `span`: sorted
// positions per work range. Top-k picks are distinct per token, so with logits (T <= span) every
// expert is one range; caller ids may repeat an expert within a token, and an expert with more
// than `span` assignments then gets ceil(cnt / span) ranges, numbered by a wave scan over the
// active experts (the multi-wave sort's records, element for element).
template <int LDT, int G>
__device__ __forceinline__ void route_small_wave(const void* logits, int T, int E, int k, int renorm,
                                                 const int32_t* ids_in, const int64_t* e2s,
                                                 int64_t num_slots, int span, SmallRouteLds& sc,
                                                 const SmallRouteOut& a, const SmallRouteOut& b) {
  constexpr int TPW = kWave / G;  // tokens per pass
  const int lane = lane_id();
  const int N = T * k;
  const int64_t my_slot = lane < E ? e2s[lane] : -1;
  int e = -2;
  if (logits != nullptr) {
    const int passes = (T + TPW - 1) / TPW;
    // every pass's loads are issued (in bounds: load_logits clamps) before any is waited for
    float v[kSmallRoutePasses][1];
#pragma unroll
    for (int ps = 0; ps < kSmallRoutePasses; ++ps)
      load_logits<LDT, G, 1>(logits, ps * TPW + lane / G, T, E, v[ps]);
#pragma unroll
    for (int ps = 0; ps < kSmallRoutePasses; ++ps) {
      if (ps >= passes) break;
      float pv = v[ps][0];
      float w;
      int id, slot;
      group_topk_select<G>(pv, E, k, renorm != 0, w, id, slot);
      const int t = ps * TPW + lane / G;
      if (t < T && slot >= 0) {
        const int f = t * k + slot;
        if (a.w) a.w[f] = w;
        if (a.ids) a.ids[f] = id;
        if (b.w) b.w[f] = w;
        if (b.ids) b.ids[f] = id;
        sc.ids[f] = id;
      }
    }
    __builtin_amdgcn_wave_barrier();
    if (lane < N) e = sc.ids[lane];
  } else if (lane < N) {
    const int x = ids_in[lane];
    e = (x >= 0 && x < E) ? x : -2;
  }
  sc.slot[lane] = (my_slot >= 0 && my_slot < num_slots) ? my_slot : -1;
  __builtin_amdgcn_wave_barrier();
  const int64_t sl = e >= 0 ? sc.slot[e] : -1;
  const bool ok = e >= 0 && sl >= 0;
  const uint64_t okm = ballot(ok);
  const bool bad = ballot(lane < N && !ok) != 0;
  if (lane < T) {
    const int32_t tm = static_cast<int32_t>((okm >> (lane * k)) & ((1ull << k) - 1));
    if (a.tmask) a.tmask[lane] = tm;
    if (b.tmask) b.tmask[lane] = tm;
  }
  const int nbits = E > 1 ? 32 - __clz(E - 1) : 0;
  uint64_t eq = okm, less = 0;
  for (int bb = nbits - 1; bb >= 0; --bb) {
    const bool bit = ok && ((e >> bb) & 1);
    const uint64_t m1 = ballot(bit);
    if (bit) less |= eq & ~m1;
    eq &= bit ? m1 : (okm & ~m1);
  }
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
  const int rank = __popcll(eq & below);
  const int nless = __popcll(less);
  const uint64_t first = ballot(ok && rank == 0);
  const bool lead = ok && rank == 0;  // this lane writes its expert's records
  const int cnt = __popcll(eq);
  const int ai = __popcll(less & first);
  const int nr = lead ? (cnt <= span ? 1 : (cnt + span - 1) / span) : 0;
  int j0 = ai;
  int nranges = __popcll(first);
  if (ballot(nr > 1) != 0) {  // wave-uniform: some expert needs several ranges
    if (lead) sc.nr[ai] = nr;
    __builtin_amdgcn_wave_barrier();
    const int v = lane < nranges ? sc.nr[lane] : 0;
    const int incl = wave_incl_scan(v);
    nranges = last_lane(incl);
    __builtin_amdgcn_wave_barrier();
    sc.nr[lane] = incl - v;  // first range of active expert `lane`
    __builtin_amdgcn_wave_barrier();
    if (lead) j0 = sc.nr[ai];
  }
  if (ok) {
    const int pos = nless + rank;
    if (a.sorted_f) a.sorted_f[pos] = lane;
    if (b.sorted_f) b.sorted_f[pos] = lane;
    if (a.fpos) { a.fpos[lane] = pos; a.fslot[lane] = sl; }
    if (b.fpos) { b.fpos[lane] = pos; b.fslot[lane] = sl; }
    if (lead) {
      RangeRec rec{};
      rec.slot = sl;
      rec.off = nless;
      rec.cnt = cnt;
      rec.key = e;
      rec.j0 = j0;
      rec.nr = nr;
      for (int r = 0; r < nr; ++r) {
        if (a.ranges) a.ranges[j0 + r] = rec;
        if (b.ranges) b.ranges[j0 + r] = rec;
      }
    }
  }
  if (lane == 0) {
    if (a.hdr) {
      a.hdr[0] = nranges;
      a.hdr[1] = bad ? 1 : 0;
      a.hdr[kHdrSingleRanges] = nranges == __popcll(first) ? 1 : 0;
    }
    if (b.hdr) {
      b.hdr[0] = nranges;
      b.hdr[1] = bad ? 1 : 0;
      b.hdr[kHdrSingleRanges] = nranges == __popcll(first) ? 1 : 0;
    }
  }
}

}  // namespace smx
