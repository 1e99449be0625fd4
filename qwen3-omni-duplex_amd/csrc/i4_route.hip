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
// TT tokens per workgroup column.  Lane l covers h = 8l + 512i.  With NORM
// every wave computes r = 1 / sqrt(mean(x^2) + eps) for its tokens in the
// same order (so all waves agree bit for bit), and wave 0 of column 0
// writes xn for the expert kernels.
template <int XT, int TT, bool NORM>
__global__ __launch_bounds__(256) void k_router_logits(
    const uint16_t* __restrict__ x, int T, int H, const uint16_t* __restrict__ wr, int E,
    const uint16_t* __restrict__ nw, float eps, uint16_t* __restrict__ xn_out,
    uint16_t* __restrict__ logits) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int e = blockIdx.x * 4 + wave;
  const int t0 = blockIdx.y * TT;
  if (e >= E) return;
  float r[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) r[t] = 1.f;
  if constexpr (NORM) {
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      float ss = 0.f;
      if (t0 + t < T)
        for (int h = 8 * lane; h < H; h += 512) ss += sumsq8<XT>(ldg16(x + (int64_t)(t0 + t) * H + h));
      ss = group_sum<64>(ss);
      r[t] = 1.0f / sqrtf(ss / (float)H + eps);
    }
  }
  const bool write_xn = NORM && xn_out != nullptr && blockIdx.x == 0 && wave == 0;
  float acc[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) acc[t] = 0.f;
  const uint16_t* wrow = wr + (int64_t)e * H;
  for (int h = 8 * lane; h < H; h += 512) {
    const u32x4 wv = ldg16(wrow + h);
    u32x4 gv = u32x4{0u, 0u, 0u, 0u};
    if constexpr (NORM) gv = ldg16(nw + h);
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      if (t0 + t < T) {
        u32x4 xv = ldg16(x + (int64_t)(t0 + t) * H + h);
        if constexpr (NORM) {
          xv.x = norm_pair<XT>(xv.x, gv.x, r[t]);
          xv.y = norm_pair<XT>(xv.y, gv.y, r[t]);
          xv.z = norm_pair<XT>(xv.z, gv.z, r[t]);
          xv.w = norm_pair<XT>(xv.w, gv.w, r[t]);
          if (write_xn) *(u32x4*)(xn_out + (int64_t)(t0 + t) * H + h) = xv;
        }
        float a = acc[t];
        a = Half<XT>::dot2(wv.x, xv.x, a);
        a = Half<XT>::dot2(wv.y, xv.y, a);
        a = Half<XT>::dot2(wv.z, xv.z, a);
        a = Half<XT>::dot2(wv.w, xv.w, a);
        acc[t] = a;
      }
    }
  }
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    const float s = group_sum<64>(acc[t]);
    if (lane == 0 && t0 + t < T) logits[(int64_t)(t0 + t) * E + e] = Half<XT>::from_f32(s);
  }
}

struct Cand {
  float v;
  int i;
};
__device__ inline bool better(Cand a, Cand b) { return a.v > b.v || (a.v == b.v && a.i < b.i); }

template <int LT> __device__ inline float load_logit(const void* p, int64_t i) {
  if constexpr (LT == I4_F32) return ((const float*)p)[i];
  else return Half<LT>::to_f32(((const uint16_t*)p)[i]);
}

// one wave per token, E <= 64 * VPL
template <int LT, int VPL>
__global__ __launch_bounds__(256) void k_topk(const void* __restrict__ logits, int T, int E,
                                              int topk, int renorm, int32_t* __restrict__ sel,
                                              float* __restrict__ wf, void* __restrict__ wh,
                                              int wht) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
  float v[VPL];
  unsigned taken = 0;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int e = lane + 64 * i;
    v[i] = e < E ? load_logit<LT>(logits, (int64_t)t * E + e) : -__builtin_inff();
    if (e >= E) taken |= 1u << i;  // padding never competes
  }
  int my_sel = 0;
  float my_val = 0.f, top_val = 0.f;
  for (int r = 0; r < topk; ++r) {
    Cand b{-__builtin_inff(), 0x7fffffff};
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const Cand c{v[i], lane + 64 * i};
      if (!((taken >> i) & 1u) && (b.i == 0x7fffffff || better(c, b))) b = c;
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
      Cand o;
      o.v = __shfl_xor(b.v, m, 64);
      o.i = __shfl_xor(b.i, m, 64);
      if (o.i != 0x7fffffff && (b.i == 0x7fffffff || better(o, b))) b = o;
    }
    if ((b.i & 63) == lane) taken |= 1u << (b.i >> 6);
    if (r == 0) top_val = b.v;
    if (lane == r) {
      my_sel = b.i;
      my_val = b.v;
    }
  }
  // softmax denominator over all E logits, max = top-1 logit
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i)
    if (lane + 64 * i < E) s += expf(v[i] - top_val);
  s = group_sum<64>(s);
  float p = lane < topk ? expf(my_val - top_val) / s : 0.f;
  if (renorm) {
    const float ps = group_sum<64>(p);
    p = p / ps;
  }
  if (lane < topk) {
    const int64_t o = (int64_t)t * topk + lane;
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
    if (xt == I4_F16) launch_router_t<I4_F16, 1>(grid, s, x, T, H, wr, E, norm_w, eps, xn, logits);
    else launch_router_t<I4_BF16, 1>(grid, s, x, T, H, wr, E, norm_w, eps, xn, logits);
  } else {
    grid.y = (T + 3) / 4;
    if (xt == I4_F16) launch_router_t<I4_F16, 4>(grid, s, x, T, H, wr, E, norm_w, eps, xn, logits);
    else launch_router_t<I4_BF16, 4>(grid, s, x, T, H, wr, E, norm_w, eps, xn, logits);
  }
  return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;
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
  if (T < 1 || T > 65535 * 4 || H < 8 || H % 8 != 0 || E < 1 || E > 65535 * 4)
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
