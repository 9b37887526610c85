// Device-side building blocks shared by the routing and expert kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace smx {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

enum DType : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

__host__ __device__ constexpr int dtype_bytes(int dt) { return dt == kF32 ? 4 : 2; }

// ---------------------------------------------------------------------------------------
// Scalar conversions. bf16 is carried as its 16-bit pattern; float->bf16 rounds to nearest
// even (NaN stays NaN), the same rule the oracle applies.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));  // v_cvt_f16_f32: nearest even
}

// Element traits: storage type, conversions, and the MFMA that consumes one 16-byte fragment
// per lane (bf16/f16: one v_mfma_f32_16x16x32; f32: four v_mfma_f32_16x16x4).
template <int DT> struct Elem;

template <> struct Elem<kBF16> {
  using S = uint16_t;
  static constexpr int kVec = 8;  // elements per 16-byte lane fragment
  __device__ static float load(const S* p) { return bf16_to_f32(*p); }
  __device__ static float to_f32(S v) { return bf16_to_f32(v); }
  __device__ static S from_f32(float f) { return f32_to_bf16(f); }
  __device__ static float round(float f) { return bf16_to_f32(f32_to_bf16(f)); }
  __device__ static f32x4 mfma(const u32x4& a, const u32x4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

template <> struct Elem<kF16> {
  using S = uint16_t;
  static constexpr int kVec = 8;
  __device__ static float load(const S* p) { return f16_to_f32(*p); }
  __device__ static float to_f32(S v) { return f16_to_f32(v); }
  __device__ static S from_f32(float f) { return f32_to_f16(f); }
  __device__ static float round(float f) { return f16_to_f32(f32_to_f16(f)); }
  __device__ static f32x4 mfma(const u32x4& a, const u32x4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

template <> struct Elem<kF32> {
  using S = float;
  static constexpr int kVec = 4;
  __device__ static float load(const S* p) { return *p; }
  __device__ static float to_f32(S v) { return v; }
  __device__ static S from_f32(float f) { return f; }
  __device__ static float round(float f) { return f; }
  __device__ static f32x4 mfma(const u32x4& a, const u32x4& b, f32x4 c) {
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.x), __uint_as_float(b.x), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.y), __uint_as_float(b.y), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.z), __uint_as_float(b.z), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.w), __uint_as_float(b.w), c, 0, 0, 0);
    return c;
  }
};

// Logit loader for any input dtype.
template <int DT> __device__ __forceinline__ float load_as_f32(const void* base, int64_t i);
template <> __device__ __forceinline__ float load_as_f32<kF32>(const void* base, int64_t i) {
  return static_cast<const float*>(base)[i];
}
template <> __device__ __forceinline__ float load_as_f32<kF16>(const void* base, int64_t i) {
  return f16_to_f32(static_cast<const uint16_t*>(base)[i]);
}
template <> __device__ __forceinline__ float load_as_f32<kBF16>(const void* base, int64_t i) {
  return bf16_to_f32(static_cast<const uint16_t*>(base)[i]);
}

// ---------------------------------------------------------------------------------------
// exp(d) for d <= 0, bit-reproducible on the CPU with plain IEEE fp32 multiply/add.
// Method: Cody & Waite argument reduction (W. J. Cody, W. Waite, "Software Manual for the
// Elementary Functions", 1980): n = rint(d*log2(e)), r = (d - n*C1) - n*C2 with
// C1 + C2 = ln 2 and C1 holding 9 significant bits so n*C1 and d - n*C1 are exact; then the
// degree-7 Taylor polynomial of e^r on |r| <= ln2/2 (truncation < 1e-8 relative), Horner
// form; then an exact scale by 2^n. Inputs below -80 return 0 so every result, and every
// softmax probability built from it, stays a normal number. Constants are fixed by their
// bit patterns. Contraction into FMA is disabled so each operation rounds once.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ float exp_nonpos(float d) {
#pragma clang fp contract(off)
  if (!(d >= -80.0f)) return d != d ? d : 0.0f;  // NaN propagates; tiny -> 0
  const float kLog2e = __uint_as_float(0x3fb8aa3bu);  // 1.44269502f
  const float kC1 = __uint_as_float(0x3f318000u);     // 0.693359375
  const float kC2 = __uint_as_float(0xb95e8083u);     // -2.12194440e-4
  const float n = rintf(d * kLog2e);
  const float r = (d - n * kC1) - n * kC2;
  float p = __uint_as_float(0x39500d01u);             // 1/5040
  p = p * r + __uint_as_float(0x3ab60b61u);           // 1/720
  p = p * r + __uint_as_float(0x3c088889u);           // 1/120
  p = p * r + __uint_as_float(0x3d2aaaabu);           // 1/24
  p = p * r + __uint_as_float(0x3e2aaaabu);           // 1/6
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  const float scale = __uint_as_float(static_cast<uint32_t>(static_cast<int>(n) + 127) << 23);
  return p * scale;
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }

// Inclusive prefix sum over the 64 lanes of a wave by DPP (VALU operand modifiers, no LDS
// round trip): row_shr 1, 2, 4, 8 within each row of 16 lanes, then row_bcast:15 adds row 0's
// (row 2's) total to rows 1 (3), and row_bcast:31 adds the first 32 lanes' total to rows 2
// and 3. Lanes whose DPP source is outside the row, or whose row is masked, add 0.
__device__ __forceinline__ int wave_incl_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15 -> rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31 -> rows 2, 3
  return v;
}

// Value of lane 63 (a wave-uniform scalar).
__device__ __forceinline__ int last_lane(int v) { return __builtin_amdgcn_readlane(v, kWave - 1); }

// c / d for 0 <= c < 2^23 and d >= 1, with rd = 1.0f / d: the float quotient is within one of
// the integer quotient, and one correction step makes it exact (a few VALU operations instead
// of an integer division's ~30).
__device__ __forceinline__ int div_small(int c, int d, float rd) {
  int q = static_cast<int>(static_cast<float>(c) * rd);
  const int r = c - q * d;
  if (r < 0) --q;
  else if (r >= d) ++q;
  return q;
}

// Wave index within the workgroup, in a scalar register: the compiler cannot see that
// threadIdx.x / 64 is the same across a wave, and values derived from it (buffer offsets)
// would otherwise be treated as per-lane.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x / kWave); }

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

// s_waitcnt immediate that waits until at most n vector-memory operations are outstanding
// (the expcnt and lgkmcnt fields at their maxima: no wait on them).
constexpr int vmcnt_imm(int n) { return (n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14); }

}  // namespace smx
