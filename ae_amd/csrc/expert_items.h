// Device helpers of the expert kernels: buffer resources, the workgroup barrier, the K-walk
// rotation, output stores and the work-item decode.
#pragma once

#include "smx_kernels.h"

namespace smx {

constexpr int kBufDword3 = 0x00020000;            // gfx9 raw-buffer resource word 3
constexpr int kNonTemporal = 2;                   // cache-policy bit: streaming (read once)
constexpr int kDeviceScope = 16;                  // cache-policy bit: device scope (sc1)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), kBufDword3);
}

// Workgroup barrier ordering LDS only: in-flight global loads stay in flight.
__device__ __forceinline__ void wg_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Order in which a workgroup walks its K chunks: step c reads chunk (c + rot) mod n. The
// accumulation order over K is then a fixed rotation per workgroup (deterministic run to run).
struct ChunkOrder {
  int n, rot;
  int base = 0;  // first chunk of the walk (a K split walks chunks base .. base + n - 1)
  __device__ __forceinline__ int at(int c) const {
    const int p = c + rot;
    return base + (p >= n ? p - n : p);
  }
};

// Gate/up workgroups start their K walk at different chunks. W1/W3 rows have a pitch of H
// elements, a power of two in bytes for the common hidden sizes (4096 and 8192 bytes in
// bf16): workgroups that sit at the same chunk at the same moment, as they do when they start
// together, then stream addresses that agree in their low 12-13 bits. Rotating the start by
// (weight-group index) / 4 measured 5.6 -> 6.1 TB/s on the H = 2048 gate/up stream and 6.3 ->
// 6.7 TB/s on H = 4096 (other rotations tried: index mod n, which keeps each XCD's workgroups
// on a few residues, was slower than none at H = 4096). The down projection's rows (pitch I)
// are walked in order: its K splits already start at different chunks, and rotating them
// measured no gain.
// (index >> 2) < 2^23 for every launch: index < (experts + 1) * (workgroups per item)
// + workgroups per item (the index of a routed item is (expert + 1) * (its expert's
// workgroups per item) + its weight group: known before the routing). The modulo is taken with a float reciprocal (div_small): a runtime
// integer division costs ~20 dependent VALU steps, on every workgroup's path to its first load.
__device__ __forceinline__ ChunkOrder rotated_order(int n, int index) {
  const int q = index >> 2;
  return ChunkOrder{n, q - div_small(q, n, 1.0f / static_cast<float>(n)) * n};
}

// The library's accurate expf (not the fast __expf): silu's value then differs from a correctly
// rounded one by about an ulp, so the rounding of act to the activation dtype rarely flips
// against the reference's arithmetic (one flipped act element moves every output of its term).
__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + expf(-g)); }

// Rounding of a routed GEMM output (gate/up, and the weighted down output): to the activation
// dtype; for fp32 runs with f16out set, to fp16 -- the reference's Triton kernel stores fp32
// runs' GEMM outputs with compute_type fp16 (specmoe/layers/fused_moe_kernel.py:203,248).
template <int DT>
__device__ __forceinline__ float round_out(float v, int f16out) {
  if constexpr (DT == kF32) return f16out ? Elem<kF16>::round(v) : v;
  else return Elem<DT>::round(v);
}

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

// store4 with device-scope stores (relaxed atomic stores at agent scope: written through to the
// level every XCD reads from). Once the wave's vector-memory counter is zero they are visible
// to device-scope loads on any XCD. idx is a multiple of 4 (8-byte aligned in 16-bit types).
template <int DT>
__device__ __forceinline__ void store4_agent(void* base, int64_t idx, float v0, float v1, float v2,
                                             float v3) {
  using S = typename Elem<DT>::S;
  auto put = [](void* p, uint64_t v) {
    __hip_atomic_store(static_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  if constexpr (DT == kF32) {
    float* p = static_cast<float*>(base) + idx;
    put(p, static_cast<uint64_t>(__float_as_uint(v0)) | (static_cast<uint64_t>(__float_as_uint(v1)) << 32));
    put(p + 2, static_cast<uint64_t>(__float_as_uint(v2)) | (static_cast<uint64_t>(__float_as_uint(v3)) << 32));
  } else {
    const uint64_t v = static_cast<uint64_t>(Elem<DT>::from_f32(v0)) |
                       (static_cast<uint64_t>(Elem<DT>::from_f32(v1)) << 16) |
                       (static_cast<uint64_t>(Elem<DT>::from_f32(v2)) << 32) |
                       (static_cast<uint64_t>(Elem<DT>::from_f32(v3)) << 48);
    put(static_cast<S*>(base) + idx, v);
  }
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ int64_t uniform64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(v) >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// The work item of one workgroup: an expert page and a list of m token rows starting at
// position `off` (routed: sorted positions, token = sorted_f / k; shared expert: token rows
// off.. directly). `tg` is the workgroup's index among the item's workgroups; `rot` is the
// index the K-walk rotation derives from -- the same for every token range of one expert, so
// that ranges streaming the same rows side by side read them in the same order.
struct WorkItem {
  const char* page;
  int64_t page_bytes;
  int I;
  int off, m, tg, rot;
  int nr;  // token ranges of the item's expert (1: its weights are read by this item only)
  bool shared;
};

// Leading `sh.*_blocks` workgroups run the shared expert (v = token range, then tg); the rest
// run the routing's work ranges (j = range, then tg). Returns false for a workgroup past the
// ranges of this batch.
// hdr and ranges: the routing's records (global memory, or a workgroup's own copy in LDS).
// W: waves per workgroup (a workgroup covers W weight tiles of its item). The K-walk rotation
// index is that of the 4-wave workgroup covering the same tiles (rot_items: workgroups per
// item at 4 waves), so the accumulation order of every output does not depend on W.
// b: the work item's index in the launch (the workgroup index, or for a workgroup that walks
// several items, the item it is on).
// Item `local` of the nr * per_item items of one expert's nr token ranges -> (range r, weight
// group g), numbered so that the nr ranges of weight group g are 8 items apart: workgroups are
// dealt to the 8 XCDs round robin, so they run on one XCD, side by side, and share its L2 for
// the rows they all read. Groups past the last multiple of 8 are numbered the same way with
// their own count as the spacing.
__device__ __forceinline__ void range_group(int local, int per_item, int nr, int& r, int& g) {
  const int full = per_item / 8 * 8 * nr;
  if (local < full) {
    const int blk = local / (8 * nr);
    const int in = local - blk * 8 * nr;
    r = in / 8;
    g = blk * 8 + (in - r * 8);
  } else {
    const int rem = per_item % 8;
    const int in = local - full;
    r = in / rem;
    g = per_item / 8 * 8 + (in - r * rem);
  }
}

// XCD order of the routed items (kByXcd): when every active expert is one range
// (hdr[kHdrSingleRanges]), at least kXcdMinRanges ranges and 8 items per range, the workgroups b
// = x mod 8 (dealt to XCD x) run ranges x, x + 8, ... whole, and the ranges past the last
// multiple of 8 item by item across the XCDs: an expert's token and activation rows are then
// fetched into one XCD's L2, not eight. Measured, same box: DeepSeek-V2-Lite 128 tokens 200.2 ->
// 197.2 us per layer, its 26-layer stack 5231 -> 5177 us; Qwen1.5-MoE 128 tokens 197.7 -> 195.5,
// 64 tokens 186.7 -> 185.1. With 8 experts (Mixtral) one page per XCD streamed slower (32
// tokens, gate/up 280 -> 295 us), hence the range minimum.
// Item q of XCD x (q = its index among the routed b = x mod 8) is range 8m + x, group g
// (q = m * per_item + g) for q < (R/8) * per_item, else item (q - (R/8) * per_item) * 8 + x of
// the remaining ranges. Every routed item below R * per_item is taken once when the launch's
// items (`nitems`: its grid, or the item count of a grid walking items 8k apart) hold at least 8
// routed items past them: XCD x then has at least ceil(R * per_item / 8) routed items, and it
// needs at most that many.
constexpr int kXcdMinRanges = 32;

__device__ __forceinline__ bool xcd_order_applies(int single, int nranges, int per_item, int nitems,
                                                  int shared_blocks) {
  return single != 0 && nranges >= kXcdMinRanges && per_item >= 8 &&
         nitems - shared_blocks - nranges * per_item >= 8;
}

// Routed item b -> (range j, weight group g) in XCD order (xcd_order_applies holds).
__device__ __forceinline__ void xcd_order(int b, int shared_blocks, int per_item, int nranges, int& j,
                                          int& g) {
  const float rpi = 1.0f / static_cast<float>(per_item);
  const int x = b & 7;
  const int first = shared_blocks + (((x - shared_blocks) % 8) + 8) % 8;
  const int q = (b - first) >> 3;
  const int full = (nranges >> 3) * per_item;
  if (q < full) {
    const int m = div_small(q, per_item, rpi);
    g = q - m * per_item;
    j = 8 * m + x;
  } else {
    const int r = (q - full) * 8 + x;
    const int m = div_small(r, per_item, rpi);
    g = r - m * per_item;
    j = (nranges & ~7) + m;
  }
}

template <typename S, int W = kExpertWaves, bool kByXcd = false>
__device__ __forceinline__ bool work_item(const ExpertArgs& a, int b, int shared_blocks, int per_item,
                                          int rot_items, WorkItem& w, const int32_t* hdr,
                                          const RangeRec* ranges, int nitems = 0) {
  const int64_t elem = static_cast<int64_t>(sizeof(S));
  const float rpi = 1.0f / static_cast<float>(per_item);  // grids hold fewer than 2^23 workgroups
  if (b < shared_blocks) {
    // The shared expert's token ranges all read its whole page: with several, they are numbered
    // like a routed expert's ranges (range_group) and load with normal caching (nr > 1).
    const int nr = a.sh.tok_groups > 1 ? a.sh.tok_groups : 1;
    int v, g;
    if (nr > 1) {
      range_group(b, per_item, nr, v, g);
    } else {
      v = div_small(b, per_item, rpi);
      g = b - v * per_item;
    }
    const int span = a.rb.span;
    w.page = static_cast<const char*>(a.sh.page);
    w.page_bytes = 3 * static_cast<int64_t>(a.H) * a.sh.I * elem;
    w.I = a.sh.I;
    w.off = v * span;
    w.m = min(span, a.T - w.off);
    w.tg = g;
    w.rot = g * W / kExpertWaves;
    w.nr = nr;
    w.shared = true;
    return true;
  }
  const int rb = b - shared_blocks;
  int j = div_small(rb, per_item, rpi);  // one of the expert's ranges; uniform across the workgroup
  // j is below the launch's range bound, so the record may be read before the range count is
  // known (the loads then share one latency); records past the count are unused.
  const int nranges = uniform(hdr[0]);
  bool by_xcd = false;
  int gx = 0;
  if constexpr (kByXcd) {
    if (xcd_order_applies(uniform(hdr[kHdrSingleRanges]), nranges, per_item,
                          nitems > 0 ? nitems : static_cast<int>(gridDim.x), shared_blocks)) {
      by_xcd = true;
      xcd_order(b, shared_blocks, per_item, nranges, j, gx);
      if (j >= nranges) return false;
    }
  }
  const RangeRec& rr = ranges[j];
  const int off = uniform(rr.off);
  const int cnt = uniform(rr.cnt);
  const int key = uniform(rr.key);
  const int j0 = uniform(rr.j0);
  const int nr = max(uniform(rr.nr), 1);
  const int64_t slot = uniform64(rr.slot);
  // the expert's nr * per_item items (range_group)
  const int local = rb - j0 * per_item;
  int g = by_xcd ? gx : local, r = 0;
  if (!by_xcd && nr > 1) range_group(local, per_item, nr, r, g);
  w.off = off + r * a.rb.span;
  w.m = min(a.rb.span, cnt - r * a.rb.span);
  w.page_bytes = a.page_elems * elem;
  w.page = static_cast<const char*>(a.pool) + slot * w.page_bytes;
  w.I = a.I;
  w.tg = g;
  w.rot = (key + 1) * rot_items + g * W / kExpertWaves;
  w.nr = nr;
  w.shared = false;
  return j < nranges;
}

template <typename S, bool kByXcd = false>
__device__ __forceinline__ bool work_item(const ExpertArgs& a, int shared_blocks, int per_item,
                                          WorkItem& w, const int32_t* hdr, const RangeRec* ranges) {
  return work_item<S, kExpertWaves, kByXcd>(a, static_cast<int>(blockIdx.x), shared_blocks, per_item,
                                            per_item, w, hdr, ranges);
}

// Routed items in expert order, for the in-launch routing when every expert is one token range
// (T <= span): item b >= shared_blocks is weight group g of expert e, b - shared_blocks =
// e * per_item + g, whether or not e has tokens; shared items as work_item. The rotation is
// work_item's (the records' key is the expert index). by_expert == nullptr (before the
// routing): the item's page, I and rotation from the expert-to-slot map -- false when e has
// no valid slot (the routing then gives it no tokens either). Otherwise by_expert[e] is the
// routing's record of expert e (every e < E, cnt 0 without routable assignments): also the
// token range -- false when it is empty.
template <typename S, int W>
__device__ __forceinline__ bool expert_item(const ExpertArgs& a, int b, int shared_blocks, int per_item,
                                            int rot_items, WorkItem& w, const RangeRec* by_expert) {
  if (b < shared_blocks)
    return work_item<S, W, false>(a, b, shared_blocks, per_item, rot_items, w, nullptr, nullptr);
  const int rb = b - shared_blocks;
  const int e = div_small(rb, per_item, 1.0f / static_cast<float>(per_item));
  const int g = rb - e * per_item;
  int64_t slot;
  if (by_expert == nullptr) {
    slot = a.e2s[e];
    if (slot < 0 || slot >= a.rt.num_slots) return false;
    w.off = 0;
    w.m = 0;
  } else {
    const RangeRec& rr = by_expert[e];
    const int cnt = uniform(rr.cnt);
    if (cnt == 0) return false;
    slot = uniform64(rr.slot);
    w.off = uniform(rr.off);
    w.m = cnt;
  }
  w.page_bytes = a.page_elems * static_cast<int64_t>(sizeof(S));
  w.page = static_cast<const char*>(a.pool) + slot * w.page_bytes;
  w.I = a.I;
  w.tg = g;
  w.rot = (e + 1) * rot_items + g * W / kExpertWaves;
  w.nr = 1;
  w.shared = false;
  return true;
}

}  // namespace smx
