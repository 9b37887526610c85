// C++ restatement of the MoE layer on the host CPU -- a timed CPU baseline. MEASUREMENT AND TEST
// INFRASTRUCTURE, NOT PRODUCT CODE: only bench.py's cpu_baseline leg (as the thing timed) and
// tests/ (which pin it against the numpy oracle, oracle/moe_ref.py) load it. The product path
// (ae_amd) never does and has no CPU fallback.
//
// The reference has no CPU expert path (FusedMoE.forward_cpu, specmoe/layers/FusedMoE.py:210-240,
// is unreachable); its one CPU kernel is attention, specmoe/csrc/flashattention.cpp, whose
// :163-207 run each contraction as one cblas_sgemm and the independent work under OpenMP. This
// file writes the MoE layer the same way: stack_fused_moe (specmoe/layers/fused_moe_kernel.py:
// 253-349) after select_experts (specmoe/layers/FusedMoE.py:174-185), per call
//
//   routing   fp32 softmax over the experts, top-k by repeated arg-max (ties to the lower expert
//             index), optional w / sum(w) in pick order;
//   experts   per active expert e, its assignments f = t*k + j in ascending order, rows x_t
//             gathered into X_e:  G = round(X_e W1_e^T), U = round(X_e W3_e^T)   (:332-335, :203)
//                                 A = round(silu(G) * U)                           (:337)
//                                 c3[t, j] = round((A W2_e^T)[row] * w[t, j])      (:339-342)
//             (three products per expert, each as one cblas_sgemm per OpenMP thread on its
//             slice of the output columns, MKL sequential inside);
//   combine   y = round(sum_j c3[:, j]), fp32, j in order                          (:344-347).
//
// round() is to bf16 (round to nearest even) for bf16 layers and nothing for fp32 ones. Weights
// arrive as fp32 matrices per expert (W1, W3 [I, H], W2 [H, I], row-major), converted once by the
// caller before any timing. The exp of the softmax and of silu is the C library's expf, so
// weights can differ from the oracle's bit-exact routing in the last ulp; ids agree unless two
// experts' probabilities are that close.
//
// MKL comes from libmkl_rt (mkl.h is not installed): the CBLAS prototype is declared here. The
// caller selects MKL's sequential layer (MKL_THREADING_LAYER=SEQUENTIAL) before the first call,
// so that the only threads are this file's OpenMP ones.
#include <omp.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

extern "C" {
enum CblasLayout { kCblasRowMajor = 101 };
enum CblasTranspose { kCblasNoTrans = 111, kCblasTrans = 112 };
void cblas_sgemm(int layout, int trans_a, int trans_b, int m, int n, int k, float alpha, const float* a,
                 int lda, const float* b, int ldb, float beta, float* c, int ldc);
}

namespace {

inline float round_bf16(float v) {
  uint32_t u;
  std::memcpy(&u, &v, 4);
  if ((u & 0x7f800000u) == 0x7f800000u) {
    if (u & 0x007fffffu) u |= 0x00400000u;  // NaN stays a quiet NaN
  } else {
    u += 0x7fffu + ((u >> 16) & 1u);
  }
  u &= 0xffff0000u;
  float r;
  std::memcpy(&r, &u, 4);
  return r;
}

inline float rnd(float v, int bf16) { return bf16 ? round_bf16(v) : v; }

inline float silu(float g) { return g / (1.0f + std::exp(-g)); }

// C [n, N] = A [n, K] . B [N, K]^T (row-major), the N columns split across the OpenMP threads in
// slices of whole 16-column groups, one sequential cblas_sgemm each.
void gemm_nt(int n, int N, int K, const float* a, const float* b, float* c) {
#pragma omp parallel
  {
    const int nt = omp_get_num_threads(), id = omp_get_thread_num();
    const int groups = (N + 15) / 16;
    const int g0 = static_cast<int>(static_cast<int64_t>(groups) * id / nt);
    const int g1 = static_cast<int>(static_cast<int64_t>(groups) * (id + 1) / nt);
    const int c0 = g0 * 16, c1 = g1 * 16 < N ? g1 * 16 : N;
    if (c1 > c0)
      cblas_sgemm(kCblasRowMajor, kCblasNoTrans, kCblasTrans, n, c1 - c0, K, 1.0f, a, K,
                  b + static_cast<int64_t>(c0) * K, K, 0.0f, c + c0, N);
  }
}

}  // namespace

extern "C" {

// y [T, H] fp32 (values in the layer's dtype); topk_w [T, k], topk_ids [T, k] out. w1, w3, w2:
// E pointers to fp32 matrices, null for an expert without a pool page (its assignments add
// nothing). bf16 != 0 rounds at the bf16 points. threads > 0 sets the OpenMP thread count.
// Returns 0, or 1 for bad arguments.
int cpu_moe_forward(const float* x, int T, int H, int I, int E, int k, const float* logits, int renorm,
                    const float* const* w1, const float* const* w3, const float* const* w2, int bf16,
                    int threads, float* y, float* topk_w, int32_t* topk_ids) {
  if (T < 0 || H <= 0 || I <= 0 || E <= 0 || k <= 0 || k > E || !x || !logits || !y || !topk_w || !topk_ids)
    return 1;
  if (threads > 0) omp_set_num_threads(threads);
  // routing
#pragma omp parallel for schedule(static)
  for (int t = 0; t < T; ++t) {
    const float* lg = logits + static_cast<int64_t>(t) * E;
    std::vector<float> p(E);
    float m = lg[0];
    for (int e = 1; e < E; ++e) m = std::fmax(m, lg[e]);
    float s = 0.0f;
    for (int e = 0; e < E; ++e) {
      p[e] = std::exp(lg[e] - m);
      s += p[e];
    }
    const float inv = 1.0f / s;
    for (int e = 0; e < E; ++e) p[e] *= inv;
    // rank: a NaN probability below every number, a picked expert below that (so every round
    // picks an expert in [0, E))
    std::vector<float> rank(p);
    for (int e = 0; e < E; ++e)
      if (!(rank[e] >= 0.0f)) rank[e] = -0.5f;
    float sum = 0.0f;
    for (int j = 0; j < k; ++j) {
      int best = 0;
      for (int e = 1; e < E; ++e)
        if (rank[e] > rank[best]) best = e;
      topk_ids[static_cast<int64_t>(t) * k + j] = best;
      topk_w[static_cast<int64_t>(t) * k + j] = p[best];
      sum = (j == 0) ? p[best] : sum + p[best];
      rank[best] = -1.0f;
    }
    if (renorm)
      for (int j = 0; j < k; ++j) topk_w[static_cast<int64_t>(t) * k + j] /= sum;
  }
  // assignments grouped by expert, ascending f within each
  const int N = T * k;
  std::vector<int> count(E + 1, 0), order(N);
  for (int f = 0; f < N; ++f) ++count[topk_ids[f] + 1];
  for (int e = 0; e < E; ++e) count[e + 1] += count[e];
  {
    std::vector<int> pos(count.begin(), count.end() - 1);
    for (int f = 0; f < N; ++f) order[pos[topk_ids[f]]++] = f;
  }
  std::vector<float> c3(static_cast<size_t>(N) * H, 0.0f);
  std::vector<float> xe, g, u, c;
  for (int e = 0; e < E; ++e) {
    const int n = count[e + 1] - count[e];
    if (n == 0 || !w1[e] || !w3[e] || !w2[e]) continue;
    const int* fs = order.data() + count[e];
    xe.resize(static_cast<size_t>(n) * H);
    g.resize(static_cast<size_t>(n) * I);
    u.resize(static_cast<size_t>(n) * I);
    c.resize(static_cast<size_t>(n) * H);
#pragma omp parallel for schedule(static)
    for (int r = 0; r < n; ++r)
      std::memcpy(&xe[static_cast<size_t>(r) * H], x + static_cast<int64_t>(fs[r] / k) * H, sizeof(float) * H);
    gemm_nt(n, I, H, xe.data(), w1[e], g.data());
    gemm_nt(n, I, H, xe.data(), w3[e], u.data());
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < static_cast<int64_t>(n) * I; ++i)
      g[i] = rnd(silu(rnd(g[i], bf16)) * rnd(u[i], bf16), bf16);
    gemm_nt(n, H, I, g.data(), w2[e], c.data());
#pragma omp parallel for schedule(static)
    for (int r = 0; r < n; ++r) {
      const float w = topk_w[fs[r]];
      float* dst = &c3[static_cast<size_t>(fs[r]) * H];
      const float* src = &c[static_cast<size_t>(r) * H];
      for (int h = 0; h < H; ++h) dst[h] = rnd(src[h] * w, bf16);
    }
  }
#pragma omp parallel for schedule(static)
  for (int t = 0; t < T; ++t) {
    float* out = y + static_cast<int64_t>(t) * H;
    const float* base = &c3[static_cast<size_t>(t) * k * H];
    for (int h = 0; h < H; ++h) {
      float s = base[h];
      for (int j = 1; j < k; ++j) s += base[static_cast<size_t>(j) * H + h];
      out[h] = rnd(s, bf16);
    }
  }
  return 0;
}

}  // extern "C"
