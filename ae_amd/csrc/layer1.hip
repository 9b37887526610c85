// The single-launch MoE layer for one token: gate/up, down projection and combine in one grid.
//
// At one token a DeepSeek-V2-Lite or Qwen1.5-MoE block reads ~138 MB of expert weights: 92 MB
// of gate/up rows, then 46 MB of down rows that need the gate/up results. As two launches the
// down rows cannot start before the last gate/up workgroup ends, and the launch boundary, the
// gate/up launch's drain and the down launch's ramp cost a fifth of the layer. Here the down
// workgroups follow the gate/up workgroups in the same grid and stream their W2 rows into
// registers while gate/up runs; only the final dot products wait for the activation rows.
//
// Grid: [gate/up workgroups 0 .. gu_blocks-1][down workgroups: one per 4 output rows]. The
// gate/up workgroups are gateup_kernel's (routing inside, one wave; 4 waves per workgroup)
// with two changes: activation rows are stored at device scope (written through), and after
// every store of the workgroup has completed, thread 0 stores the call's epoch in the
// workgroup's flag (gateup_device.h).
//
// A down workgroup (wave w: output row h = 4 * (its index) + w):
//   1. wave 0 routes the token into LDS (route_small_wave: the same top-k and records as the
//      gate/up workgroups compute);
//   2. every wave issues W2 row h of the shared expert and of each routed expert into
//      registers (at most kLayerMaxUnits 1 KB units per wave), all loads before any wait --
//      while the gate/up workgroups stream, HBM serves both;
//   3. wave 0 polls the gate/up flags with device-scope loads until each holds the epoch, or
//      until the wait bound passes (wall clock, s_memrealtime); no barrier inside the poll;
//   4. the workgroup reads the activation rows with device-scope loads into LDS;
//   5. each wave sums its terms exactly as down_rows_kernel does (per lane over 1 KB units in
//      K order, then the fixed cross-lane reduction; terms rounded and added in j order; the
//      block form), and stores y[0, h].
// A down workgroup that gives up writes NaN to its outputs and the epoch to the status word.
//
// Why no wait can deadlock: every workgroup a down workgroup waits for has a lower index, the
// hardware dispatches each XCD's share of a grid in index order, and a gate/up workgroup waits
// for nothing outside itself; so every gate/up workgroup is dispatched before any down
// workgroup of its XCD and finishes. The wait bound turns any violation of that premise into a
// loud error (NaN outputs, status word), not a hang.
//
// Reference: the launches this replaces at one token -- fused_moe_kernel (gate/up), silu_and_mul,
// fused_moe_kernel (down with MUL_ROUTED_WEIGHT) and the torch.sum combine of stack_fused_moe
// (specmoe/layers/fused_moe_kernel.py:329-347), after select_experts (FusedMoE.py:174-185).
#include "gateup_device.h"
#include "rows_device.h"

namespace smx {

constexpr int kLayerMaxTerms = 1 + kMaxTopK;  // one token: the shared term and k routed terms
constexpr int kLayerFlagLoads = kLayerMaxGuBlocks / kWave;  // flags per lane of the polling wave
constexpr int kLayerActLoads = kLayerMaxActBytes / 16 / (kExpertWaves * kWave);  // per thread

// Device-scope 8-byte load (a relaxed atomic load at agent scope: not served by a cache that
// another XCD's stores bypass).
__device__ __forceinline__ uint64_t load_agent(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int DT, int RG, int W>
__device__ void layer_down_role(const ExpertArgs& a, u32x4* stage) {
  using S = typename Elem<DT>::S;
  __shared__ SmallRouteLds sc;
  __shared__ float w_l[kWave];
  __shared__ int32_t fpos_l[kWave];
  __shared__ int64_t fslot_l[kWave];
  __shared__ int32_t tmask_l[1];
  __shared__ uint64_t term_w[kLayerMaxTerms];
  __shared__ float vals[W][kLayerMaxTerms];
  __shared__ int ok_l;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = wave_id();
  const int h = (static_cast<int>(blockIdx.x) - a.ls.gu_blocks) * W + wave;
  const int k = a.k;
  const bool shared = a.sh.I > 0;
  const bool gated = a.lo.block && shared && a.lo.sgate != nullptr;
  const int rowb = a.I * static_cast<int>(sizeof(S));
  const int units = (rowb + kRowsUnit - 1) / kRowsUnit;
  const int rowb_s = shared ? a.sh.I * static_cast<int>(sizeof(S)) : 0;
  const int units_s = (rowb_s + kRowsUnit - 1) / kRowsUnit;
  const uint64_t page_bytes = static_cast<uint64_t>(a.page_elems) * sizeof(S);
  // activation rows in LDS: the shared row, then the routed rows by sorted position
  const int act_r0 = (rowb_s + 15) / 16 * 16;

  // 1. the token's routing, by wave 0, into LDS
  if (wave == 0) {
    if (lane < k) fpos_l[lane] = -1;
    SmallRouteOut l;
    l.w = w_l;
    l.tmask = tmask_l;
    l.fpos = fpos_l;
    l.fslot = fslot_l;
    route_small_wave<DT, RG>(a.rt.logits, 1, a.rt.E, k, a.rt.renorm, a.rt.ids_in, a.e2s,
                             a.rt.num_slots, a.rb.span, sc, SmallRouteOut{}, l);
  }
  __syncthreads();
  // Term table (row 0 of each term's W2): term 0 the shared expert, term 1 + p the routed
  // assignment at sorted position p.
  const uint32_t m = static_cast<uint32_t>(tmask_l[0]);
  const uint64_t w2_off = 2ull * static_cast<uint64_t>(a.H);  // W2 follows W1 and W3
  if (tid == 0) term_w[0] = reinterpret_cast<uint64_t>(a.sh.page) + w2_off * static_cast<uint64_t>(rowb_s);
  if (tid < k && ((m >> tid) & 1u))
    term_w[1 + fpos_l[tid]] = reinterpret_cast<uint64_t>(a.pool) + static_cast<uint64_t>(fslot_l[tid]) * page_bytes +
                              w2_off * static_cast<uint64_t>(rowb);
  const int nr = __popc(m & ((1u << k) - 1u));  // routed terms (sorted positions 0 .. nr-1)
  __syncthreads();

  // 2. W2 row h of every term into registers: unit i is unit u of term tau, units of the shared
  //    term first; indices past the last unit load it again (unused). No branches: every load
  //    is issued before any is waited for.
  const int total = units_s + nr * units;
  const float rcp_units = 1.0f / static_cast<float>(units);
  u32x4 wr[kLayerMaxUnits];
  if (total > 0) {  // (0: no shared expert and every assignment dropped -- nothing to load)
#pragma unroll
    for (int i = 0; i < kLayerMaxUnits; ++i) {
      const int ii = min(i, total - 1);
      const int j = ii - units_s;
      const int r = j < 0 ? -1 : div_small(j, units, rcp_units);
      const int u = j < 0 ? ii : j - r * units;
      const int trowb = j < 0 ? rowb_s : rowb;
      const int o = min(u * kRowsUnit + lane * 16, trowb - 16);
      const uint64_t base = static_cast<uint64_t>(uniform64(static_cast<int64_t>(term_w[1 + r])));
      wr[i] = load16<kNonTemporal>(base + static_cast<uint64_t>(h) * static_cast<uint64_t>(trowb) +
                                   static_cast<uint64_t>(o));
    }
  }

  // 3. wave 0 waits for every gate/up workgroup's publication (bounded in wall-clock time);
  //    each poll has all of its flag loads in flight at once
  if (wave == 0) {
    const uint64_t t0 = wall_clock64();
    bool done = false;
    for (;;) {
      uint64_t v[kLayerFlagLoads];
#pragma unroll
      for (int i = 0; i < kLayerFlagLoads; ++i) {
        v[i] = load_agent(a.ls.flags + min(lane + i * kWave, a.ls.gu_blocks - 1));
      }
      bool mine = true;
#pragma unroll
      for (int i = 0; i < kLayerFlagLoads; ++i) mine = mine && v[i] == a.ls.epoch;
      if (ballot(!mine) == 0) {
        done = true;
        break;
      }
      if (static_cast<int64_t>(wall_clock64() - t0) > a.ls.wait_ticks) break;
      __builtin_amdgcn_s_sleep(1);
    }
    if (lane == 0) ok_l = done ? 1 : 0;
  }
  __syncthreads();
  if (!ok_l) {
    if (lane == 0) {
      static_cast<S*>(a.lo.y)[h] = Elem<DT>::from_f32(__builtin_nanf(""));
      if (wave == 0)
        __hip_atomic_store(a.ls.status, a.ls.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return;
  }

  // 4. the activation rows into LDS with device-scope 16-byte loads (all of a thread's loads in
  //    flight at once): the shared row, then routed rows 0 .. nr-1
  {
    const int ns = rowb_s / 16;
    const int n = ns + nr * rowb / 16;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.sh.act, static_cast<uint32_t>(rowb_s));
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.act, static_cast<uint32_t>(nr * rowb));
    u32x4 v[kLayerActLoads];
#pragma unroll
    for (int i = 0; i < kLayerActLoads; ++i) {
      const int q = tid + i * W * kWave;
      if (q < ns) v[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, q * 16, 0, kDeviceScope);
      else if (q < n) v[i] = __builtin_amdgcn_raw_buffer_load_b128(rr, (q - ns) * 16, 0, kDeviceScope);
    }
#pragma unroll
    for (int i = 0; i < kLayerActLoads; ++i) {
      const int q = tid + i * W * kWave;
      if (q < ns) stage[q] = v[i];
      else if (q < n) stage[act_r0 / 16 + (q - ns)] = v[i];
    }
  }
  __syncthreads();

  // 5. the wave's terms (shared term 0, routed terms 1 .. nr), down_rows_kernel's arithmetic
  {
    const char* sb = reinterpret_cast<const char*>(stage);
    float part = 0.0f;
#pragma unroll
    for (int i = 0; i < kLayerMaxUnits; ++i) {
      if (i < total) {
        const int j = i - units_s;
        const int r = j < 0 ? -1 : div_small(j, units, rcp_units);
        const int u = j < 0 ? i : j - r * units;
        const int trowb = j < 0 ? rowb_s : rowb;
        const int tunits = j < 0 ? units_s : units;
        const int abase = j < 0 ? 0 : act_r0 + r * rowb;
        const int o = u * kRowsUnit + lane * 16;
        if (o < trowb) part = dot16<DT>(wr[i], *reinterpret_cast<const u32x4*>(sb + abase + o), part);
        if (u == tunits - 1) {  // the term's last unit: its dot goes to LDS
          const float v = group_reduce<kWave>(part, [](float x, float y) { return x + y; });
          if (lane == 0) vals[wave][1 + r] = v;
          part = 0.0f;
        }
      }
    }
  }
  __builtin_amdgcn_wave_barrier();
  if (lane != 0) return;
  float y = 0.0f;
  for (int j = 0; j < k; ++j) {
    const int p = fpos_l[j];
    if ((m >> j) & 1u) y += round_out<DT>(vals[wave][1 + p] * w_l[j], a.f16out);
  }
  if (a.lo.block) {
    y = Elem<DT>::round(y);
    if (a.lo.scale != 1.0f) y = Elem<DT>::round(y * a.lo.scale);
    if (shared) {
      float sh = Elem<DT>::round(vals[wave][0]);
      if (gated) {
        const float z = load_scalar(a.lo.sgate, a.lo.sgate_dtype, 0);
        sh = Elem<DT>::round(Elem<DT>::round(1.0f / (1.0f + expf(-z))) * sh);
      }
      y += sh;
    }
  }
  static_cast<S*>(a.lo.y)[h] = Elem<DT>::from_f32(y);
}

template <int DT, int RG>
static void layer1_go(const ExpertArgs& a, unsigned blocks, hipStream_t s) {
  gateup_kernel<false, DT, 1, RG, false, kExpertWaves, false, false, true>
      <<<blocks, kExpertWaves * kWave, 0, s>>>(a);
}

template <int DT>
static void layer1_rg(const ExpertArgs& a, unsigned blocks, int route_g, hipStream_t s) {
  switch (route_g) {
    case 8: layer1_go<DT, 8>(a, blocks, s); break;
    case 16: layer1_go<DT, 16>(a, blocks, s); break;
    case 32: layer1_go<DT, 32>(a, blocks, s); break;
    default: layer1_go<DT, 64>(a, blocks, s); break;
  }
}

hipError_t launch_layer1(int dtype, const ExpertArgs& a, int max_ranges, int route_g, hipStream_t s) {
  // the limits the kernel assumes (the host plan checks them before choosing this form)
  const int64_t eb = dtype_bytes(dtype);
  const int64_t units = (a.I * eb + kRowsUnit - 1) / kRowsUnit;
  const int64_t units_s = (static_cast<int64_t>(a.sh.I) * eb + kRowsUnit - 1) / kRowsUnit;
  const int64_t act_bytes = (static_cast<int64_t>(a.sh.I) * eb + 15) / 16 * 16 + a.k * a.I * eb;
  const int64_t stage_bytes = static_cast<int64_t>(kExpertWaves) * 2 * kTileSlots * 16;
  if (a.T != 1 || a.gu_waves != kExpertWaves || a.gu_ks != 0 || a.rt.E > kWave || a.k > kWave ||
      units_s + a.k * units > kLayerMaxUnits || act_bytes > kLayerMaxActBytes || act_bytes > stage_bytes ||
      (a.I * eb) % 16 != 0 || (static_cast<int64_t>(a.sh.I) * eb) % 16 != 0 || a.H % kExpertWaves != 0 ||
      (route_g != 8 && route_g != 16 && route_g != 32 && route_g != 64) || a.ls.flags == nullptr ||
      a.ls.status == nullptr || a.ls.epoch == 0)
    return hipErrorInvalidValue;
  const int64_t groups = (a.I / kRowTile + kExpertWaves - 1) / kExpertWaves;
  const int64_t gu = a.sh.gateup_blocks + static_cast<int64_t>(max_ranges) * groups;
  if (gu != a.ls.gu_blocks || gu > kLayerMaxGuBlocks) return hipErrorInvalidValue;
  const unsigned blocks = static_cast<unsigned>(gu + a.H / kExpertWaves);
  switch (dtype) {
    case kF32: layer1_rg<kF32>(a, blocks, route_g, s); break;
    case kF16: layer1_rg<kF16>(a, blocks, route_g, s); break;
    default: layer1_rg<kBF16>(a, blocks, route_g, s); break;
  }
  return hipGetLastError();
}

}  // namespace smx
