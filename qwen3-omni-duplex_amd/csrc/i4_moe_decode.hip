// Decode (T = 1) expert kernels of the fused MoE block on I4_LAYOUT_TILE
// weights (replace the per-token loop body of FusedPackedMoE.forward,
// src/duplex/streaming/fused_packed_moe.py:231-263).
//
// k_tile_gate_up: one workgroup per (16-row block of the FFN dimension,
// selected expert): the gate tile rows n0..n0+15 and the up tile rows
// I+n0..I+n0+15, wave w walking superchunks w, w+4, ...  silu(g) * u happens
// in registers and only the half-precision activation [topk][I] is written
// (the reference writes fp32 [8][1536] and runs split / silu / mul / cast as
// separate kernels, fused_packed_moe.py:255-257).  In ROUTE mode every wave
// first ranks the logits itself and takes the expert of its slot, so routing
// costs no launch of its own; workgroup (0, 0) stores sel / w for the down
// stage.
//
// k_tile_down_m1: one workgroup per 16 output rows across ALL selected
// experts (wave w owns slots w, w+4, ...), so the routing-weighted combine and
// the residual add happen in LDS in a fixed slot order: no atomics, the
// result is bit-reproducible run to run.
#include "i4_launch.h"
#include "i4_moe_launch.h"
#include "i4_tile.h"
#include "i4_topk.h"

namespace i4 {

enum { GU_SEL = 0, GU_ROUTE = 1 };

template <int XT, int ST, bool GB, int SPW, int MODE>
__global__ __launch_bounds__(256) void k_tile_gate_up(
    const uint16_t* __restrict__ x, int topk, int32_t* __restrict__ sel,
    const uint16_t* __restrict__ logits, int E_r, int renorm, float* __restrict__ wts, TW w,
    int I, uint16_t* __restrict__ act, int32_t* __restrict__ status) {
  extern __shared__ __align__(16) unsigned char lds[];
  __shared__ float red[4][32];
  if (status && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *status = I4_OK;
  const int H = w.K, C = H >> 5, SC = H >> 7;
  u32x4* xs = (u32x4*)lds;
  float2* sums = (float2*)(lds + (size_t)H * 2);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, ln = lane & 15, kb = lane >> 4;

  const u32 mg = magic_v<XT>();
  TStager<XT> st(1, H);
  auto row_of = [&](int) -> const uint16_t* { return x; };
  int e;
  if constexpr (MODE == GU_ROUTE) {
    // the logits are the critical path: load them before the activations
    auto route = [&](auto vpl) -> int {
      constexpr int VPL = decltype(vpl)::value;
      u32 raw[VPL];
      load_row<XT, VPL>(logits, 0, E_r, raw);
      st.issue(row_of, 0);
      if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x < 64) {
        int my_sel = 0;
        float my_w = 0.f;
        topk_row<XT, VPL>(raw, 0, E_r, topk, renorm, sel, wts, nullptr, 0, &my_sel, &my_w);
        return __builtin_amdgcn_readlane(my_sel, 0);
      }
      return topk_slot<XT, VPL>(raw, E_r, blockIdx.y);
    };
    e = E_r <= 128 ? route(std::integral_constant<int, 2>{})
                   : route(std::integral_constant<int, 8>{});
  } else {
    st.issue(row_of, 0);
    e = sel[blockIdx.y];
  }
  const bool ev = (unsigned)e < (unsigned)w.E;
  const int ee = ev ? e : 0;
  const TileRow rg = tile_row<ST>(w, ee, blockIdx.x, ln, kb);
  const TileRow ru = tile_row<ST>(w, ee, (I >> 4) + blockIdx.x, ln, kb);
  TSlot<GB> sg[SPW], su[SPW];
#pragma unroll
  for (int i = 0; i < SPW; ++i) {  // clamped: the same number of loads on every path
    const int s = min(wave + 4 * i, SC - 1);
    sg[i] = tile_load<ST, GB>(rg, s, w.gshift);
    su[i] = tile_load<ST, GB>(ru, s, w.gshift);
  }
  st.commit(0, xs, sums);
  st.rest(row_of, xs, sums);
  __syncthreads();
  const u32x4* xj = xs + kb * C;
  const float2* sj = sums + kb * C;
  float ag = 0.f, au = 0.f;
#pragma unroll
  for (int i = 0; i < SPW; ++i) {
    const int s = wave + 4 * i;
    if (s < SC) {
      ag += tile_dot<XT, ST, GB>(sg[i], xj, sj, s, w.gshift, mg);
      au += tile_dot<XT, ST, GB>(su[i], xj, sj, s, w.gshift, mg);
    }
  }
  ag = kgroup_sum(ag);
  au = kgroup_sum(au);
  if (kb == 0) {
    red[wave][ln] = ag;
    red[wave][16 + ln] = au;
  }
  __syncthreads();
  if (threadIdx.x < 16) {
    const int r = threadIdx.x;
    const float g = ((red[0][r] + red[1][r]) + red[2][r]) + red[3][r];
    const float u = ((red[0][16 + r] + red[1][16 + r]) + red[2][16 + r]) + red[3][16 + r];
    act[(int64_t)blockIdx.y * I + 16 * blockIdx.x + r] =
        Half<XT>::from_f32(ev ? silu(g) * u : __builtin_nanf(""));
  }
}

// down projection + routing-weighted combine + residual (T = 1); wave w owns
// slots w + 4 jj (jj < JMAX), SCB superchunks of each per round
template <int XT, int ST, bool GB, int JMAX, int SCB>
__global__ __launch_bounds__(256) void k_tile_down_m1(
    const uint16_t* __restrict__ act, int topk, const int32_t* __restrict__ sel,
    const float* __restrict__ wts, TW w, const uint16_t* __restrict__ residual,
    uint16_t* __restrict__ out) {
  extern __shared__ __align__(16) unsigned char lds[];
  __shared__ float red[16][16];
  __shared__ float s_w[16];
  const int I = w.K, C = I >> 5, SC = I >> 7;
  u32x4* xs = (u32x4*)lds;
  float2* sums = (float2*)(lds + (size_t)topk * I * 2);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, ln = lane & 15, kb = lane >> 4;
  // unconditional loads (clamped indices): a guarded load would be waited for
  // where its branch joins, before anything else is issued
  const float wv = wts[min((int)threadIdx.x, topk - 1)];
  const int on = 16 * blockIdx.x + (int)threadIdx.x;  // output row of the combine threads
  const uint16_t res_raw = *(residual ? residual + min(on, w.N - 1) : act);
  const u32 mg = magic_v<XT>();
  TStager<XT> st(topk, I);
  auto row_of = [&](int j) { return act + (int64_t)j * I; };
  st.issue(row_of, 0);
  TileRow rp[JMAX];
  int ej[JMAX];
#pragma unroll
  for (int jj = 0; jj < JMAX; ++jj) {
    const int j = min(wave + 4 * jj, topk - 1);
    ej[jj] = sel[j];
    rp[jj] = tile_row<ST>(w, (unsigned)ej[jj] < (unsigned)w.E ? ej[jj] : 0, blockIdx.x, ln, kb);
  }
  float acc[JMAX];
#pragma unroll
  for (int jj = 0; jj < JMAX; ++jj) acc[jj] = 0.f;
  for (int s0 = 0; s0 < SC; s0 += SCB) {
    TSlot<GB> sl[JMAX][SCB];
#pragma unroll
    for (int jj = 0; jj < JMAX; ++jj)
#pragma unroll
      for (int b = 0; b < SCB; ++b) sl[jj][b] = tile_load<ST, GB>(rp[jj], min(s0 + b, SC - 1), w.gshift);
    if (s0 == 0) {
      st.commit(0, xs, sums);
      st.rest(row_of, xs, sums);
      if ((int)threadIdx.x < topk) s_w[threadIdx.x] = wv;
      __syncthreads();
    }
#pragma unroll
    for (int jj = 0; jj < JMAX; ++jj) {
      const int j = wave + 4 * jj;
      if (j < topk) {
        const u32x4* xj = xs + (4 * j + kb) * C;
        const float2* sj = sums + (4 * j + kb) * C;
#pragma unroll
        for (int b = 0; b < SCB; ++b)
          if (s0 + b < SC) acc[jj] += tile_dot<XT, ST, GB>(sl[jj][b], xj, sj, s0 + b, w.gshift, mg);
      }
    }
  }
#pragma unroll
  for (int jj = 0; jj < JMAX; ++jj) {
    const int j = wave + 4 * jj;
    // each expert's output rounded to the activation dtype before the weighted
    // sum, as the reference's y.to(x.dtype) does (fused_packed_moe.py:262)
    const float v = Half<XT>::to_f32(Half<XT>::from_f32(kgroup_sum(acc[jj])));
    if (j < topk && kb == 0) red[j][ln] = (unsigned)ej[jj] < (unsigned)w.E ? v : __builtin_nanf("");
  }
  __syncthreads();
  if ((int)threadIdx.x < 16 && on < w.N) {
    float y = 0.f;
    for (int j = 0; j < topk; ++j) y += s_w[j] * red[j][threadIdx.x];
    out[on] = Half<XT>::from_f32((residual ? Half<XT>::to_f32(res_raw) : 0.f) + y);
  }
}

// ---------------------------------------------------------------------------
// launchers
template <int XT, int ST, bool GB, int MODE>
static int gate_up_t(const GateUpArgs& a, const TW& w, int I, hipStream_t s) {
  const int SC = w.K >> 7;
  const int spw = (SC + 3) / 4;
  const dim3 grid(I / 16, a.n_slots);
  const size_t lds = (size_t)w.K * 3;  // staged x (2 B / column) + per-word sums (1 B / column)
#define I4_GU_CASE(SPW_)                                                                     \
  if (spw <= SPW_) {                                                                         \
    hipLaunchKernelGGL((k_tile_gate_up<XT, ST, GB, SPW_, MODE>), grid, dim3(256), lds, s,    \
                       (const uint16_t*)a.x, a.topk, a.sel, (const uint16_t*)a.logits, a.E_r, \
                       a.renorm, a.wts, w, I, (uint16_t*)a.act, a.status);                   \
    return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;                          \
  }
  I4_GU_CASE(1) I4_GU_CASE(2) I4_GU_CASE(4) I4_GU_CASE(8)
#undef I4_GU_CASE
  return I4_ERR_SHAPE;
}

template <int XT, int ST, bool GB>
static int down_m1_t(const void* act, int topk, const int32_t* sel, const float* wts, const TW& w,
                     const void* residual, void* out, hipStream_t s) {
  const int SC = w.K >> 7;
  const int jmax = (topk + 3) / 4;
  const size_t lds = (size_t)topk * w.K * 3;
  const dim3 grid(w.N / 16);
#define I4_DN_CASE(JM_, SCB_)                                                                  \
  if (jmax == JM_ && (SC <= SCB_ || SCB_ == 8)) {                                              \
    hipLaunchKernelGGL((k_tile_down_m1<XT, ST, GB, JM_, SCB_>), grid, dim3(256), lds, s,       \
                       (const uint16_t*)act, topk, sel, wts, w, (const uint16_t*)residual,     \
                       (uint16_t*)out);                                                        \
    return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;                            \
  }
#define I4_DN_JM(JM_) I4_DN_CASE(JM_, 2) I4_DN_CASE(JM_, 4) I4_DN_CASE(JM_, 6) I4_DN_CASE(JM_, 8)
  I4_DN_JM(1) I4_DN_JM(2) I4_DN_JM(3) I4_DN_JM(4)
#undef I4_DN_JM
#undef I4_DN_CASE
  return I4_ERR_SHAPE;
}

template <int XT, int ST>
int launch_gate_up(const GateUpArgs& a, const TW& w, int I, hipStream_t s) {
  const bool gb = w.gshift >= 2;
  if (a.route) return gb ? gate_up_t<XT, ST, true, GU_ROUTE>(a, w, I, s)
                         : gate_up_t<XT, ST, false, GU_ROUTE>(a, w, I, s);
  return gb ? gate_up_t<XT, ST, true, GU_SEL>(a, w, I, s)
            : gate_up_t<XT, ST, false, GU_SEL>(a, w, I, s);
}

template <int XT, int ST>
int launch_down_m1(const void* act, int topk, const int32_t* sel, const float* wts, const TW& w,
                   const void* residual, void* out, hipStream_t s) {
  return w.gshift >= 2 ? down_m1_t<XT, ST, true>(act, topk, sel, wts, w, residual, out, s)
                       : down_m1_t<XT, ST, false>(act, topk, sel, wts, w, residual, out, s);
}

#define I4_INST(XT_, ST_)                                                                      \
  template int launch_gate_up<XT_, ST_>(const GateUpArgs&, const TW&, int, hipStream_t);       \
  template int launch_down_m1<XT_, ST_>(const void*, int, const int32_t*, const float*,        \
                                        const TW&, const void*, void*, hipStream_t);
I4_INST(I4_F16, I4_F32) I4_INST(I4_F16, I4_F16) I4_INST(I4_F16, I4_BF16)
I4_INST(I4_BF16, I4_F32) I4_INST(I4_BF16, I4_F16) I4_INST(I4_BF16, I4_BF16)
#undef I4_INST

}  // namespace i4
