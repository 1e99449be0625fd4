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
// folded onto +0 first so that equal values tie).  Keys are unique, so the
// k selected experts are exactly the keys at or above the k-th largest key,
// found by bisection on the key bits (kth_key): each step is one compare per
// key and a ballot count, all wave-uniform scalar work, with no cross-lane
// data movement.  fp32 logits (whose keys can tie) take k rounds of a wave
// maximum instead: the value, then the lowest id holding it.
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

// Wave-uniform k-th largest of the wave's keys (unique and nonzero where
// valid, 0 where not; 1 <= k <= number of valid keys).  MSB-first bisection:
// prefix is the largest value seen so far with at least k keys at or above
// it; the search stops as soon as exactly k keys are at or above it, and the
// smallest of those is the answer.
template <int VPL> __device__ inline u32 kth_key(const u32 (&key)[VPL], int k) {
  u32 prefix = 0;
  for (int b = 31; b >= 0; --b) {
    const u32 cand = prefix | (1u << b);
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < VPL; ++i)
      cnt += __builtin_popcountll(__builtin_amdgcn_ballot_w64(key[i] >= cand));
    if (cnt >= k) {
      prefix = cand;
      if (cnt == k) break;
    }
  }
  u32 m = 0xFFFFFFFFu;
#pragma unroll
  for (int i = 0; i < VPL; ++i)
    if (key[i] >= prefix) m = min(m, key[i]);
  return wave_min_u32(m);
}

// The k keys at or above t (t = kth_key(key, k)) in descending order: lane r
// < k returns the key of rank r, lanes >= k return 0.  The selected keys are
// gathered into lanes 0..k-1 in expert order, each counts the larger ones
// among them (its rank), and a forward permute puts it in lane rank.
template <int VPL> __device__ inline u32 sorted_top_keys(const u32 (&key)[VPL], int k, u32 t) {
  const int lane = __lane_id();
  int mine = 0, j = 0;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    uint64_t m = __builtin_amdgcn_ballot_w64(key[i] >= t);
    while (m) {
      const int l = __builtin_ctzll(m);
      const int kv = __builtin_amdgcn_readlane((int)key[i], l);
      if (lane == j) mine = kv;
      m &= m - 1;
      ++j;
    }
  }
  int rank = 0;
  for (int q = 0; q < k; ++q) rank += (u32)__builtin_amdgcn_readlane(mine, q) > (u32)mine;
  const int dst = lane < k ? rank : lane;
  const int r = __builtin_amdgcn_ds_permute(dst << 2, mine);
  return lane < k ? (u32)r : 0u;
}

template <int LT> __device__ inline float load_logit(const void* p, int64_t i) {
  if constexpr (LT == I4_F32) return ((const float*)p)[i];
  else return Half<LT>::to_f32(((const uint16_t*)p)[i]);
}

// Raw bits of one row of logits (lane l holds experts l + 64 i), loaded
// without branches (indices clamped) so that all loads are in flight at once;
// a caller can issue more loads before the keys are formed.
template <int LT, int VPL>
__device__ inline void load_row(const void* __restrict__ logits, int64_t row, int E,
                                u32 (&raw)[VPL]) {
  const int lane = __lane_id();
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int64_t o = row * E + min(lane + 64 * i, E - 1);
    if constexpr (LT == I4_F32) raw[i] = __builtin_bit_cast(u32, ((const float*)logits)[o]);
    else raw[i] = ((const uint16_t*)logits)[o];
  }
}

// Values and keys of a loaded row (invalid lanes: -inf and key 0).
template <int LT, int VPL>
__device__ inline void row_keys(const u32 (&raw)[VPL], int E, float (&v)[VPL], u32 (&key)[VPL]) {
  const int lane = __lane_id();
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int e = lane + 64 * i;
    if constexpr (LT == I4_F32) {
      v[i] = e < E ? __builtin_bit_cast(float, raw[i]) : -__builtin_inff();
      key[i] = e < E ? order32(v[i]) : 0u;
    } else {
      v[i] = e < E ? Half<LT>::to_f32((uint16_t)raw[i]) : -__builtin_inff();
      key[i] = e < E ? (order16((uint16_t)raw[i]) << 16) | (0xFFFFu - e) : 0u;
    }
  }
}

// Expert of rank `slot` (0 = largest) of a loaded row of half-precision
// logits; wave-uniform.
template <int LT, int VPL>
__device__ inline int topk_slot(const u32 (&raw)[VPL], int E, int slot) {
  static_assert(LT != I4_F32, "ranked slots need unique half-precision keys");
  float v[VPL];
  u32 key[VPL];
  row_keys<LT, VPL>(raw, E, v, key);
  return (int)(0xFFFFu - (kth_key(key, slot + 1) & 0xFFFFu));
}

// Top-k of one loaded row of E <= 64 * VPL logits by one wave; writes sel / w
// for lanes < topk (descending weight), softmax over all E in fp32, optional
// renormalisation over the selected k.
template <int LT, int VPL>
__device__ inline void topk_row(const u32 (&raw)[VPL], int64_t row, int E, int topk, int renorm,
                                int32_t* __restrict__ sel, float* __restrict__ wf,
                                void* __restrict__ wh, int wht, int* out_sel = nullptr,
                                float* out_w = nullptr) {
  const int lane = __lane_id();
  float v[VPL];
  u32 key[VPL];
  row_keys<LT, VPL>(raw, E, v, key);
  int my_sel = 0;
  float my_val = 0.f, top_val = 0.f;
  if constexpr (LT != I4_F32) {
    const u32 sk = sorted_top_keys(key, topk, kth_key(key, topk));
    if (lane < topk) {
      my_sel = (int)(0xFFFFu - (sk & 0xFFFFu));
      my_val = Half<LT>::to_f32(unorder16(sk >> 16));
    }
    top_val = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_val), 0));
  } else {
    for (int r = 0; r < topk; ++r) {
      u32 m = 0;
#pragma unroll
      for (int i = 0; i < VPL; ++i) m = max(m, key[i]);
      m = wave_max_u32(m);
      u32 cand = 0xFFFFFFFFu;  // lowest id among the lanes holding the maximum value
#pragma unroll
      for (int i = 0; i < VPL; ++i)
        if (key[i] == m && m != 0u) cand = min(cand, (u32)(lane + 64 * i));
      const int id = (int)wave_min_u32(cand);
      const float val = __builtin_bit_cast(float, (m & 0x80000000u) ? (m & 0x7FFFFFFFu) : ~m);
      if ((id & 63) == lane) key[id >> 6] = 0u;
      if (r == 0) top_val = val;
      if (lane == r) {
        my_sel = id;
        my_val = val;
      }
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

template <int LT, int VPL>
__device__ inline void wave_topk_row(const void* __restrict__ logits, int64_t row, int E, int topk,
                                     int renorm, int32_t* __restrict__ sel,
                                     float* __restrict__ wf, void* __restrict__ wh, int wht) {
  u32 raw[VPL];
  load_row<LT, VPL>(logits, row, E, raw);
  topk_row<LT, VPL>(raw, row, E, topk, renorm, sel, wf, wh, wht);
}

}  // namespace i4
