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
#include "i4_router_body.h"
#include "i4_launch.h"
#include "i4_topk.h"

namespace i4 {

// T = 1: the workgroup normalises x once (8 values per thread, x and the norm
// weights loaded ahead of the router rows), shares xn through LDS, and each
// wave dots one expert row.  The sum of squares is reduced in the same fixed
// order in every workgroup, so all of them use the same r bit for bit.
// pend[0..n_pend) (16-byte units) is filled with the pending pattern for a
// following single-launch expert stage, which polls it (n_pend = 0: none), and
// *status (when given) is cleared for the failure that stage may report.
template <int XT, bool NORM>
__global__ __launch_bounds__(256) void k_router_m1(
    const uint16_t* __restrict__ x, int H, const uint16_t* __restrict__ wr, int E,
    const uint16_t* __restrict__ nw, float eps, uint16_t* __restrict__ xn_out,
    uint16_t* __restrict__ logits, u32x4* __restrict__ pend, int n_pend,
    int32_t* __restrict__ status) {
  constexpr int RL = 8;  // 512-element rounds of a router row (H <= 4096)
  __shared__ u32x4 s_xn[512];
  __shared__ float s_ss[4];
  for (int i = blockIdx.x * 256 + (int)threadIdx.x; i < n_pend; i += gridDim.x * 256)
    pend[i] = u32x4{~0u, ~0u, ~0u, ~0u};
  if (status && blockIdx.x == 0 && threadIdx.x == 0) *status = I4_OK;
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

// T = 1 with H = 2048: one wavefront per expert row (128 workgroups at E = 128
// instead of 32), with the arithmetic of k_router_m1 bit for bit.  k_router_m1's
// 256 threads each take word t of x (8 values) for the sum of squares; here lane l
// stands in for threads l, l + 64, l + 128, l + 192 -- the same words its dot
// product needs (8 l + 512 i) -- forms their partial sums in the same order and
// reduces each group of 64 with the same wave sum, so r, the normalised words
// and the logit are those of k_router_m1.  No LDS, no barrier.
// H = 1024 (the Talker's hidden size) works the same way with lanes standing in
// for threads l and l + 64 only: k_router_m1's waves 2 and 3 hold no words and
// add zeros.
template <int XT, bool NORM, int H>
__global__ __launch_bounds__(64) void k_router_m1w(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wr, int E,
    const uint16_t* __restrict__ nw, float eps, uint16_t* __restrict__ xn_out,
    uint16_t* __restrict__ logits, u32x4* __restrict__ pend, int n_pend,
    int32_t* __restrict__ status) {
  for (int i = blockIdx.x * 64 + (int)threadIdx.x; i < n_pend; i += gridDim.x * 64)
    pend[i] = u32x4{~0u, ~0u, ~0u, ~0u};
  if (status && blockIdx.x == 0 && threadIdx.x == 0) *status = I4_OK;
  router_wave<XT, NORM, H, false>(x, wr, blockIdx.x, nw, eps, xn_out, logits);
}

// k_router_m1w for the layer after an XCD-local experts launch (k_ct_moe_m1x): the
// workgroup first completes that layer, h = residual + sum_k wts[k] ypart[k]
// (slot_sum8; workgroup 0 writes h to h_out, the layer's output and the next
// residual), then routes h.  Thread t completes word t of h into LDS, wave w forms the
// sum of squares of words 64 w .. 64 w + 63 -- the partial sum router_wave's lanes
// form for i = w -- and wave 0 routes expert blockIdx.x from the staged row with the
// arithmetic of router_finish, so the logits and the normalised row are those of
// k_router_m1w bit for bit.  Four waves share the completion's 9 H half loads
// (one wave alone: 13.4 us per stack layer against 12.8; four experts per workgroup,
// one per wave, 13.2).
template <int XT, bool NORM, int H, int KC>
__global__ __launch_bounds__(256) void k_router_m1ws(
    const uint16_t* __restrict__ res, const uint16_t* __restrict__ ypart,
    const float* __restrict__ wts, uint16_t* __restrict__ h_out,
    const uint16_t* __restrict__ wr, int E, const uint16_t* __restrict__ nw, float eps,
    uint16_t* __restrict__ xn_out, uint16_t* __restrict__ logits, u32x4* __restrict__ pend,
    int n_pend, int32_t* __restrict__ status) {
  constexpr int NR = H / 512, W = H / 8;
  static_assert(W <= 256, "one word of the row per thread");
  __shared__ u32x4 s_h[W];
  __shared__ float s_ss[4];
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  for (int i = blockIdx.x * 256 + t; i < n_pend; i += gridDim.x * 256)
    pend[i] = u32x4{~0u, ~0u, ~0u, ~0u};
  if (status && blockIdx.x == 0 && t == 0) *status = I4_OK;
  const int e = blockIdx.x;
  const bool router = wave == 0 && e < E;
  u32x4 wv[NR], gv[NR];
  if (router) {
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      wv[i] = ldg16(wr + (int64_t)e * H + 8 * lane + 512 * i);
      if constexpr (NORM) gv[i] = ldg16(nw + 8 * (lane + 64 * i));
    }
  }
  float ss = 0.f;
  if (t < W) {
    u32x4 y[KC];
#pragma unroll
    for (int k = 0; k < KC; ++k) y[k] = ldg16(ypart + (int64_t)k * H + 8 * t);
    const u32x4 rv = ldg16(res + 8 * t);
    float w[KC];
#pragma unroll
    for (int k = 0; k < KC; ++k) w[k] = wts[k];
    const u32x4 h = slot_sum8<XT, KC>(rv, y, w);
    s_h[t] = h;
    if (h_out && blockIdx.x == 0) *(u32x4*)(h_out + 8 * t) = h;
    if constexpr (NORM) ss = sumsq8<XT>(h);
  }
  if constexpr (NORM) {
    ss = group_sum<64>(ss);
    if (lane == 0) s_ss[wave] = ss;
  }
  __syncthreads();
  if (!router) return;
  u32x4 xv[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) xv[i] = s_h[lane + 64 * i];
  if constexpr (NORM) {
    const float r = 1.0f / sqrtf(((s_ss[0] + s_ss[1]) + (s_ss[2] + s_ss[3])) / (float)H + eps);
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

// The same completion alone, for the last layer: out = residual + sum_k wts[k] ypart[k],
// one 16-byte word of each row per thread.
template <int XT, int KC>
__global__ __launch_bounds__(64) void k_moe_sum_m1(const uint16_t* __restrict__ res,
                                                   const uint16_t* __restrict__ ypart,
                                                   const float* __restrict__ wts, int H,
                                                   uint16_t* __restrict__ out) {
  const int m = blockIdx.x * 64 + (int)threadIdx.x;
  if (m >= H / 8) return;
  u32x4 y[KC];
#pragma unroll
  for (int k = 0; k < KC; ++k) y[k] = ldg16(ypart + (int64_t)k * H + 8 * m);
  const u32x4 r = ldg16(res + 8 * m);
  float w[KC];
#pragma unroll
  for (int k = 0; k < KC; ++k) w[k] = wts[k];
  *(u32x4*)(out + 8 * m) = slot_sum8<XT, KC>(r, y, w);
}

// T > 1, pass 1: RMSNorm of one token per workgroup with exactly the
// arithmetic of k_router_m1 (same thread -> word map, same reduction order),
// so each token's xn is bit for bit the one it gets alone.
template <int XT>
__global__ __launch_bounds__(256) void k_rmsnorm_t(const uint16_t* __restrict__ x, int H,
                                                   const uint16_t* __restrict__ nw, float eps,
                                                   uint16_t* __restrict__ xn) {
  __shared__ float s_ss[4];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int words = H >> 3;
  const uint16_t* xr = x + (int64_t)blockIdx.x * H;
  u32x4 xv[2], gv[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int m = min((int)threadIdx.x + 256 * u, words - 1);
    xv[u] = ldg16(xr + 8 * m);
    gv[u] = ldg16(nw + 8 * m);
  }
  float ss = 0.f;
#pragma unroll
  for (int u = 0; u < 2; ++u)
    if ((int)threadIdx.x + 256 * u < words) ss += sumsq8<XT>(xv[u]);
  ss = group_sum<64>(ss);
  if (lane == 0) s_ss[wave] = ss;
  __syncthreads();
  const float r =
      1.0f / sqrtf(((s_ss[0] + s_ss[1]) + (s_ss[2] + s_ss[3])) / (float)H + eps);
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int m = (int)threadIdx.x + 256 * u;
    if (m < words) {
      u32x4 v = xv[u];
      v.x = norm_pair<XT>(v.x, gv[u].x, r);
      v.y = norm_pair<XT>(v.y, gv[u].y, r);
      v.z = norm_pair<XT>(v.z, gv[u].z, r);
      v.w = norm_pair<XT>(v.w, gv[u].w, r);
      *(u32x4*)(xn + (int64_t)blockIdx.x * H + 8 * m) = v;
    }
  }
}

// T > 1, pass 2: logits of TT tokens (staged in LDS) x 4 * EPW experts per
// workgroup.  Each logit is the per-lane dot2 chain and wave sum of
// k_router_m1, so a token's logits do not depend on the batch.  Wave w owns
// experts EPW * w .. of the tile; the TT sums of one expert are formed
// together so their wave reductions overlap.
// The body takes its tile (bx: expert group, by: token tile) and stores each finished
// logit through store(token, expert, value), from lane 0 of the wave that made it.
template <int XT, int TT, int EPW, class Store>
__device__ inline void router_t_body(int bx, int by, const uint16_t* __restrict__ x, int T, int H,
                                     const uint16_t* __restrict__ wr, int E, Store store) {
  constexpr int RL = 8;  // 512-element rounds of a router row (H <= 4096)
  extern __shared__ __align__(16) unsigned char lds[];
  u32x4* s_x = (u32x4*)lds;  // [TT][words]
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int words = H >> 3, rounds = (H + 511) / 512;
  const int t0 = by * TT, e0 = (bx * 4 + wave) * EPW;
  u32x4 wv[EPW][RL];
#pragma unroll
  for (int j = 0; j < EPW; ++j) {
    const uint16_t* wrow = wr + (int64_t)min(e0 + j, E - 1) * H;
#pragma unroll
    for (int i = 0; i < RL; ++i)
      wv[j][i] = i < rounds ? ldg16(wrow + min(8 * lane + 512 * i, H - 8)) : u32x4{0u, 0u, 0u, 0u};
  }
  // all staging loads in flight before the first LDS write (a load / wait /
  // write loop would pay one memory latency per round)
  constexpr int NS = TT * 512 / 256;  // 16-byte words per thread at H = 4096
  const int total = TT * words;
  u32x4 sv[NS];
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    if (256 * u < total) {
      const int idx = min((int)threadIdx.x + 256 * u, total - 1);
      const int tk = idx / words, m = idx - tk * words;
      sv[u] = ldg16(x + (int64_t)min(t0 + tk, T - 1) * H + 8 * m);
    }
  }
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    const int idx = (int)threadIdx.x + 256 * u;
    if (256 * u < total && idx < total) s_x[idx] = sv[u];
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < EPW; ++j) {
    float a[TT];
#pragma unroll
    for (int tk = 0; tk < TT; ++tk) {
      a[tk] = 0.f;
#pragma unroll
      for (int i = 0; i < RL; ++i) {
        const int h = 8 * lane + 512 * i;
        if (i < rounds && h < H) {
          const u32x4 xw = s_x[tk * words + (h >> 3)];
          a[tk] = Half<XT>::dot2(wv[j][i].x, xw.x, a[tk]);
          a[tk] = Half<XT>::dot2(wv[j][i].y, xw.y, a[tk]);
          a[tk] = Half<XT>::dot2(wv[j][i].z, xw.z, a[tk]);
          a[tk] = Half<XT>::dot2(wv[j][i].w, xw.w, a[tk]);
        }
      }
    }
#pragma unroll
    for (int tk = 0; tk < TT; ++tk) a[tk] = group_sum<64>(a[tk]);
    const int e = e0 + j;
    if (lane == 0 && e < E) {
#pragma unroll
      for (int tk = 0; tk < TT; ++tk)
        if (t0 + tk < T) store(t0 + tk, e, a[tk]);
    }
  }
}

template <int XT, int TT, int EPW>
__global__ __launch_bounds__(256) void k_router_t(const uint16_t* __restrict__ x, int T, int H,
                                                  const uint16_t* __restrict__ wr, int E,
                                                  uint16_t* __restrict__ logits) {
  router_t_body<XT, TT, EPW>(blockIdx.x, blockIdx.y, x, T, H, wr, E, [&](int t, int e, float a) {
    logits[(int64_t)t * E + e] = Half<XT>::from_f32(a);
  });
}

// Tag of the routing words of one call at workspace epoch e: odd, so a zero-filled
// buffer never matches.
__device__ inline u32 route_tag(u32 e) { return (2u * e + 1u) * 0x9E3779B1u; }

// Routing of 2..64 tokens (E <= 128, E % 4 == 0) as one launch.  Blocks [0, T E / 4) are
// k_router_t<XT, 1, 1>'s workgroups (block b: token b / (E / 4), experts 4 (b % (E / 4))
// .. + 3, one per wave; the same logits bit for bit); each writes its four logits as two
// (value pair, tag) words, lgt [T][E / 2][2], in one 16-byte store written through.  The
// ceil(T / 4) blocks after them rank one token per wave, as k_topk does, once every word
// of the token's row holds this call's tag (loads past the L1, at most max_polls passes:
// then the token's routing weights are NaN and I4_ERR_HANDOFF goes to *status), and set
// pend (n_pend 16-byte units) to the pending pattern for the grouped launch.  Only the
// later blocks wait, and only for earlier ones.  A later launch of the call (k_group)
// advances *epoch, so the next call's words carry another tag and no pending pattern is
// needed here.  status_reset (nullable) gets I4_OK from block 0 first.  rank_only: the
// ranking blocks alone (no router blocks; every wait then gives up), for testing the
// bounded wait from the host.
template <int XT>
__global__ __launch_bounds__(256) void k_router_topk_t(
    const uint16_t* __restrict__ x, int T, int H, const uint16_t* __restrict__ wr, int E,
    u32* lgt, const u32* __restrict__ epoch, int topk, int renorm,
    int32_t* __restrict__ sel, float* __restrict__ wf, u32x4* __restrict__ pend, int n_pend,
    int32_t* __restrict__ status_reset, int32_t* __restrict__ status, int max_polls,
    int rank_only) {
  const int G = E >> 2, nr = rank_only ? 0 : G * T;
  const int b = blockIdx.x;
  const u32 tag = route_tag(__builtin_amdgcn_readfirstlane(*epoch));
  if (b < nr) {
    __shared__ uint16_t s_lg[4];
    if (b == 0 && status_reset && threadIdx.x == 0) *status_reset = I4_OK;
    const int t = b / G, g = b - t * G;
    router_t_body<XT, 1, 1>(g, t, x, T, H, wr, E,
                            [&](int, int e, float a) { s_lg[e & 3] = Half<XT>::from_f32(a); });
    __syncthreads();
    if (threadIdx.x == 0) {
      const u32 p0 = (u32)s_lg[0] | ((u32)s_lg[1] << 16), p1 = (u32)s_lg[2] | ((u32)s_lg[3] << 16);
      const rsrc_t r = rsrc(lgt, (u32)T * (u32)E * 4u);
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{p0, tag, p1, tag}, r,
                                             (u32)t * (u32)E * 4u + (u32)g * 16u, 0, kCoherent);
    }
    return;
  }
  const int rb = b - nr, nrb = (int)gridDim.x - nr;
  for (int i = rb * 256 + (int)threadIdx.x; i < n_pend; i += nrb * 256)
    pend[i] = u32x4{~0u, ~0u, ~0u, ~0u};
  const int t = rb * 4 + ((int)threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (t >= T) return;
  // lane l ranks experts l and l + 64 (load_row's order), from words l / 2 and 32 + l / 2
  // (lgt is not __restrict__, so the reloads stay inside the wait loop)
  const rsrc_t r = rsrc(lgt, (u32)T * (u32)E * 4u);
  const int ea = min(lane, E - 1), eb = min(lane + 64, E - 1);
  const u32 ra = (u32)t * (u32)E * 4u;
  u32x2 va, vb;
  bool late = false;
  for (int it = 0;; ++it) {
    va = __builtin_amdgcn_raw_buffer_load_b64(r, ra + (u32)(ea >> 1) * 8u, 0, kCoherent);
    vb = __builtin_amdgcn_raw_buffer_load_b64(r, ra + (u32)(eb >> 1) * 8u, 0, kCoherent);
    if (__builtin_amdgcn_ballot_w64(va.y != tag || vb.y != tag) == 0) break;
    if (it >= max_polls) {
      late = true;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
    asm volatile("" ::: "memory");
  }
  u32 raw[2] = {(va.x >> (16 * (ea & 1))) & 0xFFFFu, (vb.x >> (16 * (eb & 1))) & 0xFFFFu};
  topk_row<XT, 2>(raw, t, E, topk, renorm, sel, wf, nullptr, 0);
  if (late) {
    if (lane < topk) wf[(int64_t)t * topk + lane] = __builtin_nanf("");
    if (lane == 0 && status) *status = I4_ERR_HANDOFF;
  }
}

// one wave per token; every thread also fills its share of pend (n_pend 16-byte units)
// with the pending pattern
template <int LT, int VPL>
__global__ __launch_bounds__(256) void k_topk(const void* __restrict__ logits, int T, int E,
                                              int topk, int renorm, int32_t* __restrict__ sel,
                                              float* __restrict__ wf, void* __restrict__ wh,
                                              int wht, u32x4* __restrict__ pend, int n_pend) {
  for (int i = blockIdx.x * 256 + (int)threadIdx.x; i < n_pend; i += gridDim.x * 256)
    pend[i] = u32x4{~0u, ~0u, ~0u, ~0u};
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  wave_topk_row<LT, VPL>(logits, t, E, topk, renorm, sel, wf, wh, wht);
}

}  // namespace i4

using namespace i4;

int i4_launch_router_logits(const void* x, int xt, int T, int H, const void* wr, int E,
                            const void* norm_w, float eps, void* xn, void* logits, hipStream_t s,
                            void* pend, int n_pend, int32_t* status) {
  dim3 grid((E + 3) / 4, 1);
  if (T == 1 && (H == 2048 || H == 1024)) {  // one wavefront per expert
#define I4_RM1W_CASE(XT_, N_, H_)                                                              \
  if (xt == XT_ && (norm_w != nullptr) == N_ && H == H_)                                       \
    hipLaunchKernelGGL((k_router_m1w<XT_, N_, H_>), dim3(E), dim3(64), 0, s,                   \
                       (const uint16_t*)x, (const uint16_t*)wr, E, (const uint16_t*)norm_w,    \
                       eps, (uint16_t*)xn, (uint16_t*)logits, (u32x4*)pend, n_pend, status);
    I4_RM1W_CASE(I4_F16, true, 2048) else I4_RM1W_CASE(I4_F16, false, 2048)
    else I4_RM1W_CASE(I4_BF16, true, 2048) else I4_RM1W_CASE(I4_BF16, false, 2048)
    else I4_RM1W_CASE(I4_F16, true, 1024) else I4_RM1W_CASE(I4_F16, false, 1024)
    else I4_RM1W_CASE(I4_BF16, true, 1024) else I4_RM1W_CASE(I4_BF16, false, 1024)
#undef I4_RM1W_CASE
  } else if (T == 1) {
#define I4_RM1_CASE(XT_, N_)                                                                  \
  if (xt == XT_ && (norm_w != nullptr) == N_)                                                 \
    hipLaunchKernelGGL((k_router_m1<XT_, N_>), grid, dim3(256), 0, s, (const uint16_t*)x, H,  \
                       (const uint16_t*)wr, E, (const uint16_t*)norm_w, eps, (uint16_t*)xn,   \
                       (uint16_t*)logits, (u32x4*)pend, n_pend, status);
    I4_RM1_CASE(I4_F16, true) else I4_RM1_CASE(I4_F16, false) else I4_RM1_CASE(I4_BF16, true)
    else I4_RM1_CASE(I4_BF16, false)
#undef I4_RM1_CASE
  } else {
    const uint16_t* xin = (const uint16_t*)x;
    if (norm_w) {
      if (xt == I4_F16)
        hipLaunchKernelGGL(k_rmsnorm_t<I4_F16>, dim3(T), dim3(256), 0, s, xin, H,
                           (const uint16_t*)norm_w, eps, (uint16_t*)xn);
      else
        hipLaunchKernelGGL(k_rmsnorm_t<I4_BF16>, dim3(T), dim3(256), 0, s, xin, H,
                           (const uint16_t*)norm_w, eps, (uint16_t*)xn);
      xin = (const uint16_t*)xn;
    }
    // tiles of TT tokens x 4 EPW experts: up to 64 tokens one token per tile
    // (T = 32: 1024 workgroups of few registers; 3 us faster per M = 32 layer
    // than 4-token tiles, whose 238 VGPRs allow one wave per SIMD), larger
    // batches reuse each staged token and router row more
#define I4_RT_CASE(XT_, TT_, EPW_)                                                            \
  if (xt == XT_) {                                                                            \
    const dim3 g2((E + 4 * EPW_ - 1) / (4 * EPW_), (T + TT_ - 1) / TT_);                      \
    const size_t lds = (size_t)TT_ * (H / 8) * 16; /* <= 64 KB for H <= 4096 */               \
    hipLaunchKernelGGL((k_router_t<XT_, TT_, EPW_>), g2, dim3(256), lds, s, xin, T, H,        \
                       (const uint16_t*)wr, E, (uint16_t*)logits);                            \
  }
    if (T <= 64) {
      I4_RT_CASE(I4_F16, 1, 1) else I4_RT_CASE(I4_BF16, 1, 1)
    } else {
      I4_RT_CASE(I4_F16, 8, 2) else I4_RT_CASE(I4_BF16, 8, 2)
    }
#undef I4_RT_CASE
  }
  return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;
}

int i4_launch_router_sum(const void* res, const void* ypart, const float* wts, int kc,
                         void* h_out, int xt, int H, const void* wr, int E, const void* norm_w,
                         float eps, void* xn, void* logits, hipStream_t s, void* pend,
                         int n_pend, int32_t* status) {
#define I4_RS_CASE(XT_, N_, H_)                                                                \
  if (xt == XT_ && (norm_w != nullptr) == N_ && H == H_) {                                     \
    hipLaunchKernelGGL((k_router_m1ws<XT_, N_, H_, 8>), dim3(E), dim3(256), 0, s,              \
                       (const uint16_t*)res, (const uint16_t*)ypart, wts, (uint16_t*)h_out,    \
                       (const uint16_t*)wr, E, (const uint16_t*)norm_w, eps, (uint16_t*)xn,    \
                       (uint16_t*)logits, (u32x4*)pend, n_pend, status);                       \
    return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;                            \
  }
  if (kc != 8) return I4_ERR_SHAPE;
  I4_RS_CASE(I4_F16, true, 2048) I4_RS_CASE(I4_F16, false, 2048)
  I4_RS_CASE(I4_BF16, true, 2048) I4_RS_CASE(I4_BF16, false, 2048)
  I4_RS_CASE(I4_F16, true, 1024) I4_RS_CASE(I4_F16, false, 1024)
  I4_RS_CASE(I4_BF16, true, 1024) I4_RS_CASE(I4_BF16, false, 1024)
#undef I4_RS_CASE
  return I4_ERR_SHAPE;
}

int i4_launch_moe_sum(const void* res, const void* ypart, const float* wts, int kc, int xt,
                      int H, void* out, hipStream_t s) {
  if (kc != 8 || H % 8 != 0) return I4_ERR_SHAPE;
  const dim3 grid((H / 8 + 63) / 64);
  if (xt == I4_F16)
    hipLaunchKernelGGL((k_moe_sum_m1<I4_F16, 8>), grid, dim3(64), 0, s, (const uint16_t*)res,
                       (const uint16_t*)ypart, wts, H, (uint16_t*)out);
  else
    hipLaunchKernelGGL((k_moe_sum_m1<I4_BF16, 8>), grid, dim3(64), 0, s, (const uint16_t*)res,
                       (const uint16_t*)ypart, wts, H, (uint16_t*)out);
  return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;
}

int i4_launch_topk(const void* logits, int lt, int T, int E, int topk, int renorm, int32_t* sel,
                   float* wf, void* wh, int wht, hipStream_t s, void* pend, int n_pend) {
  dim3 grid((T + 3) / 4);
#define I4_TOPK_CASE(LT_, VPL_)                                                             \
  if (lt == LT_ && E <= 64 * VPL_) {                                                        \
    hipLaunchKernelGGL((k_topk<LT_, VPL_>), grid, dim3(256), 0, s, logits, T, E, topk,      \
                       renorm, sel, wf, wh, wht, (u32x4*)pend, n_pend);                      \
    return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;                         \
  }
  I4_TOPK_CASE(I4_F16, 2) I4_TOPK_CASE(I4_F16, 8)
  I4_TOPK_CASE(I4_BF16, 2) I4_TOPK_CASE(I4_BF16, 8)
  I4_TOPK_CASE(I4_F32, 2) I4_TOPK_CASE(I4_F32, 8)
#undef I4_TOPK_CASE
  return I4_ERR_SHAPE;
}

int i4_launch_router_topk(const void* x, int xt, int T, int H, const void* wr, int E,
                          const void* norm_w, float eps, void* xn, u32* lgt, const u32* epoch,
                          int topk, int renorm, int32_t* sel, float* wf, void* pend, int n_pend,
                          int32_t* status_reset, int32_t* status, int max_polls, bool rank_only,
                          hipStream_t s) {
  if (T < 2 || T > 64 || E > 128 || E % 4 != 0 || topk > E) return I4_ERR_SHAPE;
  const uint16_t* xin = (const uint16_t*)x;
  if (norm_w) {
    if (xt == I4_F16)
      hipLaunchKernelGGL(k_rmsnorm_t<I4_F16>, dim3(T), dim3(256), 0, s, xin, H,
                         (const uint16_t*)norm_w, eps, (uint16_t*)xn);
    else
      hipLaunchKernelGGL(k_rmsnorm_t<I4_BF16>, dim3(T), dim3(256), 0, s, xin, H,
                         (const uint16_t*)norm_w, eps, (uint16_t*)xn);
    xin = (const uint16_t*)xn;
  }
  const dim3 grid((rank_only ? 0 : (E / 4) * T) + (T + 3) / 4);
  const size_t lds = (size_t)(H / 8) * 16;
#define I4_RTK_CASE(XT_)                                                                        hipLaunchKernelGGL((k_router_topk_t<XT_>), grid, dim3(256), lds, s, xin, T, H,                                  (const uint16_t*)wr, E, lgt, epoch, topk, renorm, sel, wf, (u32x4*)pend,                      n_pend, status_reset, status, max_polls, (int)rank_only)
  if (xt == I4_F16) I4_RTK_CASE(I4_F16);
  else I4_RTK_CASE(I4_BF16);
#undef I4_RTK_CASE
  return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;
}

extern "C" {

int i4_router_logits(const void* x, int x_dtype, int T, int H, const void* router_w, int E,
                     const void* norm_w, float norm_eps, void* xn_out, void* logits,
                     hipStream_t stream) {
  if (!x || !router_w || !logits) return I4_ERR_NULL;
  if (xn_out && !norm_w) return I4_ERR_NULL;
  if (norm_w && T > 1 && !xn_out) return I4_ERR_NULL;  // the norm pass writes xn there
  if (((uintptr_t)norm_w & 15) || ((uintptr_t)xn_out & 15)) return I4_ERR_ALIGN;
  if (x_dtype != I4_F16 && x_dtype != I4_BF16) return I4_ERR_DTYPE;
  if (T < 1 || T > 65535 * 4 || H < 8 || H % 8 != 0 || H > 4096 || E < 1 || E > 65535 * 4)
    return I4_ERR_SHAPE;
  if (((uintptr_t)x & 15) || ((uintptr_t)router_w & 15)) return I4_ERR_ALIGN;
  return i4_launch_router_logits(x, x_dtype, T, H, router_w, E, norm_w, norm_eps, xn_out, logits,
                                 stream);
}

int i4_rmsnorm(const void* x, int x_dtype, int T, int H, const void* norm_w, float eps, void* out,
               hipStream_t stream) {
  if (!x || !norm_w || !out) return I4_ERR_NULL;
  if (x_dtype != I4_F16 && x_dtype != I4_BF16) return I4_ERR_DTYPE;
  if (T < 1 || T > 65535 * 4 || H < 8 || H % 8 != 0 || H > 4096) return I4_ERR_SHAPE;
  if (((uintptr_t)x & 15) || ((uintptr_t)norm_w & 15) || ((uintptr_t)out & 15)) return I4_ERR_ALIGN;
  if (x_dtype == I4_F16)
    hipLaunchKernelGGL(i4::k_rmsnorm_t<I4_F16>, dim3(T), dim3(256), 0, stream,
                       (const uint16_t*)x, H, (const uint16_t*)norm_w, eps, (uint16_t*)out);
  else
    hipLaunchKernelGGL(i4::k_rmsnorm_t<I4_BF16>, dim3(T), dim3(256), 0, stream,
                       (const uint16_t*)x, H, (const uint16_t*)norm_w, eps, (uint16_t*)out);
  return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;
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
