// Router kernels: dense gate Linear (logits) and softmax / top-k / renorm.
//
// Reference: FusedPackedMoE.forward, src/duplex/streaming/fused_packed_moe.py:195-199
//   w = softmax(gate(x), dim=1, dtype=float); w, sel = topk(w, k);
//   w /= w.sum(-1); w = w.to(x.dtype)
// softmax is monotone, and distinct half-precision logits map to distinct fp32
// probabilities, so ranking the logits themselves gives the same experts as
// ranking the probabilities.  Exact ties are broken by the lower expert id
// (torch.topk leaves that order unspecified).
#include "i4_common.h"
#include "i4_launch.h"
#include "i4_topk.h"

namespace i4 {

// RMSNorm of 8 values (one 16-byte load): round(round(x * r) * w), the order
// of transformers' Qwen3OmniMoeThinkerTextRMSNorm.forward
// (modeling_qwen3_omni_moe.py:1388-1393 in transformers 5.15).
template <int XT> __device__ inline u32 norm_pair(u32 xp, u32 wp, float r) {
  const float a = Half<XT>::to_f32(Half<XT>::from_f32(Half<XT>::to_f32((uint16_t)xp) * r));
  const float b = Half<XT>::to_f32(Half<XT>::from_f32(Half<XT>::to_f32((uint16_t)(xp >> 16)) * r));
  const u32 lo = Half<XT>::from_f32(a * Half<XT>::to_f32((uint16_t)wp));
  const u32 hi = Half<XT>::from_f32(b * Half<XT>::to_f32((uint16_t)(wp >> 16)));
  return lo | (hi << 16);
}

template <int XT> __device__ inline float sumsq8(u32x4 d) {
  float s = 0.f;
  const u32 w[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a = Half<XT>::to_f32((uint16_t)w[i]), b = Half<XT>::to_f32((uint16_t)(w[i] >> 16));
    s += a * a;
    s += b * b;
  }
  return s;
}

// logits[t][e] = round(sum_h xn[t][h] * wr[e][h]); one wave per expert row,
// TT tokens per workgroup column.  Lane l covers h = 8l + 512i (H <= 2048 *
// RL).  The router-row loads are issued before the norm reduction.  With
// NORM every wave computes r = 1 / sqrt(mean(x^2) + eps) for its tokens in
// the same order (so all waves agree bit for bit), and wave 0 of column 0
// writes xn for the expert kernels.
template <int XT, int TT, bool NORM>
__device__ inline void router_rows(const uint16_t* __restrict__ x, int T, int H,
                                   const uint16_t* __restrict__ wr, int E,
                                   const uint16_t* __restrict__ nw, float eps,
                                   uint16_t* __restrict__ xn_out, uint16_t* __restrict__ logits) {
  constexpr int RL = 8;  // 512-element rounds held in registers (H <= 4096)
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int e = blockIdx.x * 4 + wave;
  const int t0 = blockIdx.y * TT;
  if (e >= E) return;
  const int rounds = (H + 511) / 512;
  const uint16_t* wrow = wr + (int64_t)e * H;
  u32x4 wv[RL];
#pragma unroll
  for (int i = 0; i < RL; ++i) {
    const int h = min(8 * lane + 512 * i, H - 8);
    wv[i] = i < rounds ? ldg16(wrow + h) : u32x4{0u, 0u, 0u, 0u};
  }
  const bool write_xn = NORM && xn_out != nullptr && blockIdx.x == 0 && wave == 0;
  u32x4 gv[RL];
  if constexpr (NORM) {  // norm weights with the router rows, ahead of any dependency
#pragma unroll
    for (int i = 0; i < RL; ++i) {
      const int h = min(8 * lane + 512 * i, H - 8);
      gv[i] = i < rounds ? ldg16(nw + h) : u32x4{0u, 0u, 0u, 0u};
    }
  }
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    if (t0 + t >= T) break;
    const uint16_t* xr = x + (int64_t)(t0 + t) * H;
    u32x4 xv[RL];
#pragma unroll
    for (int i = 0; i < RL; ++i) {
      const int h = min(8 * lane + 512 * i, H - 8);
      xv[i] = i < rounds ? ldg16(xr + h) : u32x4{0u, 0u, 0u, 0u};
    }
    if constexpr (NORM) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < RL; ++i)
        if (i < rounds && 8 * lane + 512 * i < H) ss += sumsq8<XT>(xv[i]);
      ss = group_sum<64>(ss);
      const float r = 1.0f / sqrtf(ss / (float)H + eps);
#pragma unroll
      for (int i = 0; i < RL; ++i) {
        const int h = 8 * lane + 512 * i;
        if (i < rounds && h < H) {
          xv[i].x = norm_pair<XT>(xv[i].x, gv[i].x, r);
          xv[i].y = norm_pair<XT>(xv[i].y, gv[i].y, r);
          xv[i].z = norm_pair<XT>(xv[i].z, gv[i].z, r);
          xv[i].w = norm_pair<XT>(xv[i].w, gv[i].w, r);
          if (write_xn) *(u32x4*)(xn_out + (int64_t)(t0 + t) * H + h) = xv[i];
        }
      }
    }
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < RL; ++i) {
      if (i < rounds && 8 * lane + 512 * i < H) {
        a = Half<XT>::dot2(wv[i].x, xv[i].x, a);
        a = Half<XT>::dot2(wv[i].y, xv[i].y, a);
        a = Half<XT>::dot2(wv[i].z, xv[i].z, a);
        a = Half<XT>::dot2(wv[i].w, xv[i].w, a);
      }
    }
    a = group_sum<64>(a);
    if (lane == 0) logits[(int64_t)(t0 + t) * E + e] = Half<XT>::from_f32(a);
  }
}

template <int XT, int TT, bool NORM>
__global__ __launch_bounds__(256) void k_router_logits(
    const uint16_t* __restrict__ x, int T, int H, const uint16_t* __restrict__ wr, int E,
    const uint16_t* __restrict__ nw, float eps, uint16_t* __restrict__ xn_out,
    uint16_t* __restrict__ logits) {
  router_rows<XT, TT, NORM>(x, T, H, wr, E, nw, eps, xn_out, logits);
}

// T = 1: the workgroup normalises x once (8 values per thread, x and the norm
// weights loaded ahead of the router rows), shares xn through LDS, and each
// wave dots one expert row.  The sum of squares is reduced in the same fixed
// order in every workgroup, so all of them use the same r bit for bit.
template <int XT, bool NORM>
__global__ __launch_bounds__(256) void k_router_m1(
    const uint16_t* __restrict__ x, int H, const uint16_t* __restrict__ wr, int E,
    const uint16_t* __restrict__ nw, float eps, uint16_t* __restrict__ xn_out,
    uint16_t* __restrict__ logits) {
  constexpr int RL = 8;  // 512-element rounds of a router row (H <= 4096)
  __shared__ u32x4 s_xn[512];
  __shared__ float s_ss[4];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int words = H >> 3, rounds = (H + 511) / 512;
  u32x4 xv[2], gv[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int m = min((int)threadIdx.x + 256 * u, words - 1);
    xv[u] = ldg16(x + 8 * m);
    if constexpr (NORM) gv[u] = ldg16(nw + 8 * m);
  }
  const int e = blockIdx.x * 4 + wave;
  const uint16_t* wrow = wr + (int64_t)min(e, E - 1) * H;
  u32x4 wv[RL];
#pragma unroll
  for (int i = 0; i < RL; ++i)
    wv[i] = i < rounds ? ldg16(wrow + min(8 * lane + 512 * i, H - 8)) : u32x4{0u, 0u, 0u, 0u};
  float r = 1.f;
  if constexpr (NORM) {
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < 2; ++u)
      if ((int)threadIdx.x + 256 * u < words) ss += sumsq8<XT>(xv[u]);
    ss = group_sum<64>(ss);
    if (lane == 0) s_ss[wave] = ss;
    __syncthreads();
    r = 1.0f / sqrtf(((s_ss[0] + s_ss[1]) + (s_ss[2] + s_ss[3])) / (float)H + eps);
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int m = (int)threadIdx.x + 256 * u;
    if (m < words) {
      u32x4 v = xv[u];
      if constexpr (NORM) {
        v.x = norm_pair<XT>(v.x, gv[u].x, r);
        v.y = norm_pair<XT>(v.y, gv[u].y, r);
        v.z = norm_pair<XT>(v.z, gv[u].z, r);
        v.w = norm_pair<XT>(v.w, gv[u].w, r);
        if (xn_out && blockIdx.x == 0) *(u32x4*)(xn_out + 8 * m) = v;
      }
      s_xn[m] = v;
    }
  }
  __syncthreads();
  float a = 0.f;
#pragma unroll
  for (int i = 0; i < RL; ++i) {
    const int h = 8 * lane + 512 * i;
    if (i < rounds && h < H) {
      const u32x4 xw = s_xn[h >> 3];
      a = Half<XT>::dot2(wv[i].x, xw.x, a);
      a = Half<XT>::dot2(wv[i].y, xw.y, a);
      a = Half<XT>::dot2(wv[i].z, xw.z, a);
      a = Half<XT>::dot2(wv[i].w, xw.w, a);
    }
  }
  a = group_sum<64>(a);
  if (lane == 0 && e < E) logits[e] = Half<XT>::from_f32(a);
}

// one wave per token
template <int LT, int VPL>
__global__ __launch_bounds__(256) void k_topk(const void* __restrict__ logits, int T, int E,
                                              int topk, int renorm, int32_t* __restrict__ sel,
                                              float* __restrict__ wf, void* __restrict__ wh,
                                              int wht) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  wave_topk_row<LT, VPL>(logits, t, E, topk, renorm, sel, wf, wh, wht);
}

// Router logits + top-k in one launch.  Every workgroup of token tile y
// computes 4 expert rows of logits; the last one to finish (device-scope
// counter per tile) ranks the tile's tokens and resets the counter, so the
// counters are zero again after every launch.
template <int XT, int TT, bool NORM>
__global__ __launch_bounds__(256) void k_router_topk(
    const uint16_t* __restrict__ x, int T, int H, const uint16_t* __restrict__ wr, int E,
    const uint16_t* __restrict__ nw, float eps, uint16_t* __restrict__ xn_out,
    uint16_t* __restrict__ logits, int topk, int renorm, int32_t* __restrict__ sel,
    float* __restrict__ wf, unsigned* __restrict__ counters) {
  router_rows<XT, TT, NORM>(x, T, H, wr, E, nw, eps, xn_out, logits);
  __threadfence();
  __syncthreads();
  __shared__ bool last;
  if (threadIdx.x == 0) last = atomicAdd(&counters[blockIdx.y], 1u) == gridDim.x - 1;
  __syncthreads();
  if (!last) return;
  __threadfence();
  const int wave = threadIdx.x >> 6, t = blockIdx.y * TT + wave;
  if (wave < TT && t < T) {
    if (E <= 128) wave_topk_row<XT, 2>(logits, t, E, topk, renorm, sel, wf, nullptr, 0);
    else wave_topk_row<XT, 8>(logits, t, E, topk, renorm, sel, wf, nullptr, 0);
  }
  if (threadIdx.x == 0) counters[blockIdx.y] = 0u;
}

}  // namespace i4

using namespace i4;

template <int XT, int TT>
static void launch_router_t(dim3 grid, hipStream_t s, const void* x, int T, int H, const void* wr,
                            int E, const void* nw, float eps, void* xn, void* logits) {
  if (nw)
    hipLaunchKernelGGL((k_router_logits<XT, TT, true>), grid, dim3(256), 0, s, (const uint16_t*)x,
                       T, H, (const uint16_t*)wr, E, (const uint16_t*)nw, eps, (uint16_t*)xn,
                       (uint16_t*)logits);
  else
    hipLaunchKernelGGL((k_router_logits<XT, TT, false>), grid, dim3(256), 0, s,
                       (const uint16_t*)x, T, H, (const uint16_t*)wr, E, (const uint16_t*)nullptr,
                       eps, (uint16_t*)nullptr, (uint16_t*)logits);
}

int i4_launch_router_logits(const void* x, int xt, int T, int H, const void* wr, int E,
                            const void* norm_w, float eps, void* xn, void* logits, hipStream_t s) {
  dim3 grid((E + 3) / 4, 1);
  if (T == 1) {
#define I4_RM1_CASE(XT_, N_)                                                                  \
  if (xt == XT_ && (norm_w != nullptr) == N_)                                                 \
    hipLaunchKernelGGL((k_router_m1<XT_, N_>), grid, dim3(256), 0, s, (const uint16_t*)x, H,  \
                       (const uint16_t*)wr, E, (const uint16_t*)norm_w, eps, (uint16_t*)xn,   \
                       (uint16_t*)logits);
    I4_RM1_CASE(I4_F16, true) else I4_RM1_CASE(I4_F16, false) else I4_RM1_CASE(I4_BF16, true)
    else I4_RM1_CASE(I4_BF16, false)
#undef I4_RM1_CASE
  } else {
    grid.y = (T + 3) / 4;
    if (xt == I4_F16) launch_router_t<I4_F16, 4>(grid, s, x, T, H, wr, E, norm_w, eps, xn, logits);
    else launch_router_t<I4_BF16, 4>(grid, s, x, T, H, wr, E, norm_w, eps, xn, logits);
  }
  return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;
}

int i4_launch_router_topk(const void* x, int xt, int T, int H, const void* wr, int E,
                          const void* norm_w, float eps, void* xn, void* logits, int topk,
                          int renorm, int32_t* sel, float* wf, unsigned* counters,
                          hipStream_t s) {
  const int TT = T == 1 ? 1 : 4;
  dim3 grid((E + 3) / 4, (T + TT - 1) / TT);
#define I4_RT_CASE(XT_, TT_, N_)                                                                \
  if (xt == XT_ && TT == TT_ && (norm_w != nullptr) == N_) {                                    \
    hipLaunchKernelGGL((k_router_topk<XT_, TT_, N_>), grid, dim3(256), 0, s, (const uint16_t*)x, \
                       T, H, (const uint16_t*)wr, E, (const uint16_t*)norm_w, eps,             \
                       (uint16_t*)xn, (uint16_t*)logits, topk, renorm, sel, wf, counters);     \
    return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;                             \
  }
  I4_RT_CASE(I4_F16, 1, true) I4_RT_CASE(I4_F16, 1, false) I4_RT_CASE(I4_F16, 4, true)
  I4_RT_CASE(I4_F16, 4, false) I4_RT_CASE(I4_BF16, 1, true) I4_RT_CASE(I4_BF16, 1, false)
  I4_RT_CASE(I4_BF16, 4, true) I4_RT_CASE(I4_BF16, 4, false)
#undef I4_RT_CASE
  return I4_ERR_DTYPE;
}

int i4_launch_topk(const void* logits, int lt, int T, int E, int topk, int renorm, int32_t* sel,
                   float* wf, void* wh, int wht, hipStream_t s) {
  dim3 grid((T + 3) / 4);
#define I4_TOPK_CASE(LT_, VPL_)                                                             \
  if (lt == LT_ && E <= 64 * VPL_) {                                                        \
    hipLaunchKernelGGL((k_topk<LT_, VPL_>), grid, dim3(256), 0, s, logits, T, E, topk,      \
                       renorm, sel, wf, wh, wht);                                           \
    return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;                         \
  }
  I4_TOPK_CASE(I4_F16, 2) I4_TOPK_CASE(I4_F16, 8)
  I4_TOPK_CASE(I4_BF16, 2) I4_TOPK_CASE(I4_BF16, 8)
  I4_TOPK_CASE(I4_F32, 2) I4_TOPK_CASE(I4_F32, 8)
#undef I4_TOPK_CASE
  return I4_ERR_SHAPE;
}

extern "C" {

int i4_router_logits(const void* x, int x_dtype, int T, int H, const void* router_w, int E,
                     const void* norm_w, float norm_eps, void* xn_out, void* logits,
                     hipStream_t stream) {
  if (!x || !router_w || !logits) return I4_ERR_NULL;
  if (xn_out && !norm_w) return I4_ERR_NULL;
  if (((uintptr_t)norm_w & 15) || ((uintptr_t)xn_out & 15)) return I4_ERR_ALIGN;
  if (x_dtype != I4_F16 && x_dtype != I4_BF16) return I4_ERR_DTYPE;
  if (T < 1 || T > 65535 * 4 || H < 8 || H % 8 != 0 || H > 4096 || E < 1 || E > 65535 * 4)
    return I4_ERR_SHAPE;
  if (((uintptr_t)x & 15) || ((uintptr_t)router_w & 15)) return I4_ERR_ALIGN;
  return i4_launch_router_logits(x, x_dtype, T, H, router_w, E, norm_w, norm_eps, xn_out, logits,
                                 stream);
}

int i4_route_topk(const void* logits, int logits_dtype, int T, int E, int topk, int renorm,
                  int32_t* sel, float* w_f32, void* w_half, int w_half_dtype,
                  hipStream_t stream) {
  if (!logits || !sel) return I4_ERR_NULL;
  if (logits_dtype != I4_F32 && logits_dtype != I4_F16 && logits_dtype != I4_BF16)
    return I4_ERR_DTYPE;
  if (w_half && w_half_dtype != I4_F32 && w_half_dtype != I4_F16 && w_half_dtype != I4_BF16)
    return I4_ERR_DTYPE;
  if (T < 1 || T > 65535 * 4 || E < 1 || E > 512 || topk < 1 || topk > E || topk > 64)
    return I4_ERR_SHAPE;
  return i4_launch_topk(logits, logits_dtype, T, E, topk, renorm, sel, w_f32, w_half,
                        w_half_dtype, stream);
}

}  // extern "C"
