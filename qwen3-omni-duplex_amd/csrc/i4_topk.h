// Wave-level top-k routing shared by the router and the decode expert kernels.
//
// Reference: FusedPackedMoE.forward, src/duplex/streaming/fused_packed_moe.py:195-199
//   w = softmax(gate(x), dim=1, dtype=float); w, sel = topk(w, k);
//   w /= w.sum(-1); w = w.to(x.dtype)
#pragma once

#include "i4_common.h"

namespace i4 {

// ---------------------------------------------------------------------------
// top-k.  A half-precision logit becomes a 32-bit key: its bits mapped to an
// unsigned order in the high half, 0xFFFF - id in the low half, so the
// largest key is the largest value with the lowest id among ties (-0 is
// folded onto +0 first so that equal values tie).  Each round takes the wave
// maximum (4 DPP steps inside each 16-lane row, then the 4 row results via
// v_readlane) and retires the winning key.  fp32 logits use two reductions
// per round (value, then the lowest id holding it).
__device__ inline u32 order16(uint16_t b) {
  if (b == 0x8000u) b = 0;
  return (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
}
__device__ inline uint16_t unorder16(u32 o) {
  return (uint16_t)((o & 0x8000u) ? (o & 0x7FFFu) : (~o & 0xFFFFu));
}
__device__ inline u32 order32(float f) {
  u32 b = __builtin_bit_cast(u32, f);
  if (b == 0x80000000u) b = 0;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

template <int CTRL> __device__ inline u32 dpp_u32(u32 v) {
  return (u32)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

// wave-uniform maximum of v (returned in every lane)
__device__ inline u32 wave_max_u32(u32 v) {
  v = max(v, dpp_u32<0xB1>(v));   // quad_perm [1,0,3,2]
  v = max(v, dpp_u32<0x4E>(v));   // quad_perm [2,3,0,1]
  v = max(v, dpp_u32<0x141>(v));  // row_half_mirror
  v = max(v, dpp_u32<0x140>(v));  // row_mirror
  const u32 a = (u32)__builtin_amdgcn_readlane((int)v, 0);
  const u32 b = (u32)__builtin_amdgcn_readlane((int)v, 16);
  const u32 c = (u32)__builtin_amdgcn_readlane((int)v, 32);
  const u32 d = (u32)__builtin_amdgcn_readlane((int)v, 48);
  return max(max(a, b), max(c, d));
}
__device__ inline u32 wave_min_u32(u32 v) { return ~wave_max_u32(~v); }

template <int LT> __device__ inline float load_logit(const void* p, int64_t i) {
  if constexpr (LT == I4_F32) return ((const float*)p)[i];
  else return Half<LT>::to_f32(((const uint16_t*)p)[i]);
}

// Top-k of one row of E <= 64 * VPL logits by one wave; writes sel / w for
// lanes < topk (descending weight), softmax over all E in fp32, optional
// renormalisation over the selected k.
template <int LT, int VPL>
__device__ inline void wave_topk_row(const void* __restrict__ logits, int64_t row, int E, int topk,
                                     int renorm, int32_t* __restrict__ sel,
                                     float* __restrict__ wf, void* __restrict__ wh, int wht,
                                     int* out_sel = nullptr, float* out_w = nullptr) {
  const int lane = __lane_id();
  float v[VPL];
  u32 key[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int e = lane + 64 * i;
    v[i] = e < E ? load_logit<LT>(logits, row * E + e) : -__builtin_inff();
    if constexpr (LT == I4_F32) key[i] = e < E ? order32(v[i]) : 0u;
    else key[i] = e < E ? (order16(((const uint16_t*)logits)[row * E + e]) << 16) | (0xFFFFu - e) : 0u;
  }
  int my_sel = 0;
  float my_val = 0.f, top_val = 0.f;
  for (int r = 0; r < topk; ++r) {
    u32 m = 0;
#pragma unroll
    for (int i = 0; i < VPL; ++i) m = max(m, key[i]);
    m = wave_max_u32(m);
    int id;
    float val;
    if constexpr (LT == I4_F32) {
      u32 cand = 0xFFFFFFFFu;  // lowest id among the lanes holding the maximum value
#pragma unroll
      for (int i = 0; i < VPL; ++i)
        if (key[i] == m && m != 0u) cand = min(cand, (u32)(lane + 64 * i));
      id = (int)wave_min_u32(cand);
      val = __builtin_bit_cast(float, (m & 0x80000000u) ? (m & 0x7FFFFFFFu) : ~m);
      if ((id & 63) == lane) key[id >> 6] = 0u;
    } else {
      id = (int)(0xFFFFu - (m & 0xFFFFu));
      val = Half<LT>::to_f32(unorder16(m >> 16));
#pragma unroll
      for (int i = 0; i < VPL; ++i)
        if (key[i] == m) key[i] = 0u;
    }
    if (r == 0) top_val = val;
    if (lane == r) {
      my_sel = id;
      my_val = val;
    }
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i)
    if (lane + 64 * i < E) s += expf(v[i] - top_val);
  s = group_sum<64>(s);
  float p = lane < topk ? expf(my_val - top_val) / s : 0.f;
  if (renorm) p = p / group_sum<64>(p);
  if (out_sel) {  // per-lane result: lane j < topk holds slot j
    *out_sel = my_sel;
    *out_w = p;
  }
  if (sel && lane < topk) {
    const int64_t o = row * topk + lane;
    sel[o] = my_sel;
    if (wf) wf[o] = p;
    if (wh) {
      if (wht == I4_F16) ((uint16_t*)wh)[o] = Half<I4_F16>::from_f32(p);
      else if (wht == I4_BF16) ((uint16_t*)wh)[o] = Half<I4_BF16>::from_f32(p);
      else ((float*)wh)[o] = p;
    }
  }
}

}  // namespace i4
