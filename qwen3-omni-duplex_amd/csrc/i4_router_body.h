// One router logit per wavefront at T = 1 (the body of k_router_m1w), shared by
// the router launch and by the decoder-layer launch that runs it behind the
// o_proj workgroups producing its input row.
#pragma once

#include "i4_common.h"

namespace i4 {

// Wave-uniform: does any lane hold the pending pattern in one of its NR words?
template <int NR> __device__ inline bool wave_pending(const u32x4 (&v)[NR]) {
  bool p = false;
#pragma unroll
  for (int i = 0; i < NR; ++i) p |= has_pending(v[i]);
  return __builtin_amdgcn_ballot_w64(p) != 0;
}

// The part of the router wave after its row x is in registers: RMSNorm (with NORM),
// the normalised row to xn_out (expert 0's wave), the dot with router row wv and the
// logit.  Lane l holds words l + 64 i of x, the norm weight and the router row.
template <int XT, bool NORM, int H>
__device__ __forceinline__ void router_finish(u32x4 (&xv)[H / 512], const u32x4 (&gv)[H / 512],
                                              const u32x4 (&wv)[H / 512], int e, float eps,
                                              uint16_t* __restrict__ xn_out,
                                              uint16_t* __restrict__ logits) {
  constexpr int NR = H / 512;
  const int lane = threadIdx.x & 63;
  if constexpr (NORM) {
    float ws[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NR; ++i) ws[i] = group_sum<64>(sumsq8<XT>(xv[i]));  // wave i's sum
    const float r = 1.0f / sqrtf(((ws[0] + ws[1]) + (ws[2] + ws[3])) / (float)H + eps);
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      xv[i].x = norm_pair<XT>(xv[i].x, gv[i].x, r);
      xv[i].y = norm_pair<XT>(xv[i].y, gv[i].y, r);
      xv[i].z = norm_pair<XT>(xv[i].z, gv[i].z, r);
      xv[i].w = norm_pair<XT>(xv[i].w, gv[i].w, r);
      if (xn_out && e == 0) *(u32x4*)(xn_out + 8 * (lane + 64 * i)) = xv[i];
    }
  }
  float a = 0.f;
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    a = Half<XT>::dot2(wv[i].x, xv[i].x, a);
    a = Half<XT>::dot2(wv[i].y, xv[i].y, a);
    a = Half<XT>::dot2(wv[i].z, xv[i].z, a);
    a = Half<XT>::dot2(wv[i].w, xv[i].w, a);
  }
  a = group_sum<64>(a);
  if (lane == 0) logits[e] = Half<XT>::from_f32(a);
}

// Logit of expert row e from x (H halves): with NORM, x = RMSNorm(x; nw, eps) first
// (the wave writes the normalised row to xn_out when e == 0).  Lane l owns words
// l + 64 i, i < H / 512 (k_router_m1's threads l, l + 64, ..., same partial sums in
// the same order), so the logit is that of k_router_m1 bit for bit.
// POLL: x is written by earlier workgroups of the same launch and holds the pending
// pattern until then; the wave issues its weight loads, then reads x from memory
// until no word is pending (at most max_polls times: then *late is set and the
// logit is computed from whatever was read).  x is not __restrict__ here: the memory
// clobber in the wait loop then keeps the loads inside it.
// x_copy (nullable, POLL): expert 0's wave also writes the row as it read it there.
template <int XT, bool NORM, int H, bool POLL>
__device__ __forceinline__ void router_wave(const uint16_t* x, const uint16_t* __restrict__ wr, int e,
                                   const uint16_t* __restrict__ nw, float eps,
                                   uint16_t* __restrict__ xn_out, uint16_t* __restrict__ logits,
                                   int max_polls = 0, bool* late = nullptr,
                                   uint16_t* __restrict__ x_copy = nullptr) {
  static_assert(H == 1024 || H == 2048, "one 512-value round per 64 lanes, 2 or 4 rounds");
  constexpr int NR = H / 512;  // lane l owns words l + 64 i, i < NR
  const int lane = threadIdx.x & 63;
  u32x4 xv[NR], gv[NR], wv[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    if constexpr (!POLL) xv[i] = ldg16(x + 8 * (lane + 64 * i));
    if constexpr (NORM) gv[i] = ldg16(nw + 8 * (lane + 64 * i));
    wv[i] = ldg16(wr + (int64_t)e * H + 8 * lane + 512 * i);
  }
  if constexpr (POLL) {
    const rsrc_t rx = rsrc(x, (u32)H * 2u);
    for (int it = 0;; ++it) {
#pragma unroll
      for (int i = 0; i < NR; ++i) xv[i] = ld16_coherent(rx, (u32)(lane + 64 * i) * 16u);
      if (!wave_pending<NR>(xv)) break;
      if (it >= max_polls) {
        *late = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
      asm volatile("" ::: "memory");
    }
    if (x_copy && e == 0) {
#pragma unroll
      for (int i = 0; i < NR; ++i) *(u32x4*)(x_copy + 8 * (lane + 64 * i)) = xv[i];
    }
  }
  router_finish<XT, NORM, H>(xv, gv, wv, e, eps, xn_out, logits);
}

// The routing-weighted sum that completes a decode layer whose experts left one
// output row per slot (k_ct_moe_m1x):
//   h = residual + sum_k w[k] y[k],  in fp32 in slot order, rounded once,
// for the 8 values of one 16-byte word of each row: the arithmetic of the single-launch
// combine (k_ct_moe_m1's down workgroups), so the result is equal bit for bit.
template <int XT, int KC>
__device__ __forceinline__ u32x4 slot_sum8(u32x4 res, const u32x4 (&y)[KC], const float (&w)[KC]) {
  const u32 rw[4] = {res.x, res.y, res.z, res.w};
  u32 o[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    u32 pair = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float f = 0.f;
#pragma unroll
      for (int k = 0; k < KC; ++k) {
        const u32 yw[4] = {y[k].x, y[k].y, y[k].z, y[k].w};
        f = __builtin_fmaf(w[k], Half<XT>::to_f32((uint16_t)(yw[q] >> (16 * h))), f);
      }
      const float v = Half<XT>::to_f32((uint16_t)(rw[q] >> (16 * h))) + f;
      pair |= (u32)Half<XT>::from_f32(v) << (16 * h);
    }
    o[q] = pair;
  }
  return u32x4{o[0], o[1], o[2], o[3]};
}

}  // namespace i4
