// Device pieces of the fused down projection + combine (one wave per output row): the term
// table and its cursor, the 16-byte dot and the global loads, shared by down_rows_kernel
// (experts.hip) and the down workgroups of the single-launch layer (layer1.hip), so that both
// sum every term in the same order.
#pragma once

#include "expert_items.h"

namespace smx {

// One element of a runtime-typed array, as fp32 (the shared-expert gate logits).
__device__ __forceinline__ float load_scalar(const void* base, int dtype, int64_t i) {
  switch (dtype) {
    case kF32: return load_as_f32<kF32>(base, i);
    case kF16: return load_as_f32<kF16>(base, i);
    default: return load_as_f32<kBF16>(base, i);
  }
}

constexpr int kRowsWaves = 4;                                   // rows (waves) per workgroup
constexpr int kRowsDepth = 4;                                   // units in flight per wave
constexpr int kRowsUnit = kWave * 16;                           // bytes per unit
constexpr int kRowsMaxAssign = kRowsMaxTokens * kMaxTopK;
constexpr int kRowsMaxTerms = kRowsMaxAssign + kRowsMaxTokens;
static_assert(kRowsUnit == kRowsUnitBytes, "unit size of the host-side rule");

struct RowTerm {
  uint64_t w;   // byte address of row 0 of the term's W2
  uint64_t a;   // byte address of the term's activation row
  int rowb;     // bytes per row
  int units;    // kRowsUnit units per row
};

// Wave-uniform position in the term stream: term, unit within it, and the term's row.
struct RowCursor {
  int tau, u, rowb, units;
  uint64_t w, a;
};

__device__ __forceinline__ void row_cursor_at(RowCursor& c, const RowTerm* terms, int tau, int h) {
  const RowTerm& r = terms[tau];
  c.tau = tau;
  c.u = 0;
  c.rowb = uniform(r.rowb);
  c.units = uniform(r.units);
  c.w = static_cast<uint64_t>(uniform64(static_cast<int64_t>(r.w))) +
        static_cast<uint64_t>(h) * static_cast<uint64_t>(c.rowb);
  c.a = static_cast<uint64_t>(uniform64(static_cast<int64_t>(r.a)));
}

// acc + the 16-byte lane slices' element products, in element order.
template <int DT>
__device__ __forceinline__ float dot16(const u32x4& wv, const u32x4& xv, float acc) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if constexpr (DT == kF32) {
      acc = fmaf(__uint_as_float(wv[e]), __uint_as_float(xv[e]), acc);
    } else {
      using S = typename Elem<DT>::S;
      acc = fmaf(Elem<DT>::to_f32(static_cast<S>(wv[e] & 0xffffu)),
                 Elem<DT>::to_f32(static_cast<S>(xv[e] & 0xffffu)), acc);
      acc = fmaf(Elem<DT>::to_f32(static_cast<S>(wv[e] >> 16)),
                 Elem<DT>::to_f32(static_cast<S>(xv[e] >> 16)), acc);
    }
  }
  return acc;
}

// 16-byte load from a global-memory byte address (global, not flat, instructions: their
// completion is tracked by the vector-memory counter alone).
typedef const __attribute__((address_space(1))) u32x4* GlobalU32x4;

template <int CP>
__device__ __forceinline__ u32x4 load16(uint64_t addr) {
  if constexpr (CP == kNonTemporal)
    return __builtin_nontemporal_load(reinterpret_cast<GlobalU32x4>(addr));
  else
    return *reinterpret_cast<GlobalU32x4>(addr);
}

}  // namespace smx
