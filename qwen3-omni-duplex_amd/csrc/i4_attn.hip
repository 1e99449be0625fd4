// Decode attention of the Thinker's text layers (one token), the caller of the
// int4 path: transformers Qwen3OmniMoeThinkerTextAttention.forward
// (modeling_qwen3_omni_moe.py:1473-1514 in transformers 5.15) with the
// DynamicCache of src/duplex/streaming/clock.py:164-172.  The q/k/v and o
// projections are the library's int4 GEMVs; this file holds what lies between
// them:
//   k_attn_chunk    one workgroup per (kv head, 64 cached positions): RMSNorm
//                   over head_dim (q_norm / k_norm) and the rotary embedding at
//                   `pos` for the kv head's query heads and (in the workgroup
//                   holding `pos`) this token's key, which it appends to the
//                   cache with its value (cos / sin rounded to the activation
//                   dtype and every product rounded, as transformers computes in
//                   bf16); then the scores of the query heads (GQA: each K and V
//                   row is loaded once for all of them), the chunk's softmax
//                   statistics and the probability-weighted sum of V in fp32;
//   k_attn_combine  merges the chunks of each query head (flash-decoding) and
//                   rounds the output once to the activation dtype.
// Text positions are equal along mRoPE's three axes, where the interleaved
// multimodal rotary embedding (apply_interleaved_mrope) reduces to the 1-D one
// with inv_freq[i] = theta^(-2i / head_dim).
#include "i4_common.h"
#include "i4_gemv_body.h"
#include "i4_launch.h"
#include "i4_moe_launch.h"
#include "i4_router_body.h"

namespace i4 {

static constexpr int HD = 128;    // head_dim
// cached positions per attention workgroup (32 gives 272 workgroups at the Thinker's
// context 1024 instead of 136, but measured 819 against 814 us per decode step: the
// merge's extra batch of chunk loads outweighs the shorter chunks)
static constexpr int ACH = 64;
static constexpr int GQMAX = 8;   // query heads per kv head
static constexpr int PSTR = HD + 4;  // floats per chunk partial: m, l, pad, acc[HD] at 4

struct RopeTab {
  float inv_freq[HD / 2];
};

template <int XT> __device__ inline float rnd(float v) {
  return Half<XT>::to_f32(Half<XT>::from_f32(v));
}

__device__ inline float xor32(float v) {
  const int src = ((int)__lane_id() ^ 32) << 2;
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src, __builtin_bit_cast(int, v)));
}

template <int L> __device__ inline float group_max(float v) {
  if constexpr (L >= 2) v = fmaxf(v, dpp_mov<0xB1>(v));
  if constexpr (L >= 4) v = fmaxf(v, dpp_mov<0x4E>(v));
  if constexpr (L >= 8) v = fmaxf(v, dpp_mov<0x141>(v));
  if constexpr (L >= 16) v = fmaxf(v, dpp_mov<0x140>(v));
  if constexpr (L >= 32)
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v),
                                                                        0x401F)));  // xor 16
  return v;
}

// RMSNorm over one head (lane l holds dims 2l, 2l + 1 of the 128) and the
// rotary embedding at `pos`; returns the two rounded outputs packed.
// rotate_half pairs dim d with d +- 64, i.e. lane l with lane l ^ 32.
template <int XT>
__device__ inline u32 head_norm_rope(u32 raw, u32 wraw, float eps, int pos, const RopeTab& rt) {
  const int lane = __lane_id();
  const float x0 = Half<XT>::to_f32((uint16_t)raw), x1 = Half<XT>::to_f32((uint16_t)(raw >> 16));
  const float ss = group_sum<64>(x0 * x0 + x1 * x1);
  const float r = 1.0f / sqrtf(ss / (float)HD + eps);
  const u32 n = norm_pair<XT>(raw, wraw, r);
  const float a0 = Half<XT>::to_f32((uint16_t)n), a1 = Half<XT>::to_f32((uint16_t)(n >> 16));
  const float b0 = xor32(a0), b1 = xor32(a1);  // dims 2l +- 64, 2l + 1 +- 64
  const int i0 = (2 * lane) & (HD / 2 - 1);
  const float g0 = (float)pos * rt.inv_freq[i0], g1 = (float)pos * rt.inv_freq[i0 + 1];
  const float c0 = rnd<XT>(cosf(g0)), s0 = rnd<XT>(sinf(g0));
  const float c1 = rnd<XT>(cosf(g1)), s1 = rnd<XT>(sinf(g1));
  // rotate_half(x)[d] = -x[d + 64] (d < 64), x[d - 64] (d >= 64)
  const float sg = lane < 32 ? -1.f : 1.f;
  const float o0 = rnd<XT>(rnd<XT>(a0 * c0) + rnd<XT>(sg * b0 * s0));
  const float o1 = rnd<XT>(rnd<XT>(a1 * c1) + rnd<XT>(sg * b1 * s1));
  return (u32)Half<XT>::from_f32(o0) | ((u32)Half<XT>::from_f32(o1) << 16);
}

// Workgroup (chunk c, kv head g) attends positions [64c, 64c + 64) of [0, S),
// S = pos + 1.  It issues its K and V rows first, then normalises and rotates
// the group's query heads itself from the projection output (each chunk of a
// group repeats that: 8 heads of 128 values), and the workgroup whose chunk
// holds `pos` also makes this token's key (normalised, rotated) and value,
// stores them in the cache and uses them in place of the rows it could not
// have loaded.  Scores are v_dot2 products of the rounded half-precision q and
// k pairs with fp32 accumulation; softmax statistics and P V in fp32.
// part[(c * nq + head) * PSTR] = {chunk max m, sum l, -, -, acc[HD]}.
// POLL: the q|k|v row is written by earlier workgroups of the same launch (the
// projection of k_qkv_chunk) as (value pair, tag) words, 8 bytes per two values: each
// wave first issues its K / V loads, then reads its words from memory (sc1) until every
// one carries this call's tag -- at most max_polls times; a wait that gives up makes the
// query NaN and stores I4_ERR_HANDOFF to *o_status.  qkv is then not __restrict__ (the
// loads stay inside the wait loop).
template <int XT, int GQ, bool POLL>
__device__ inline void chunk_body(
    int c, int by, const uint16_t* qkv, int nq, int nkv, const uint16_t* __restrict__ qn_w,
    const uint16_t* __restrict__ kn_w, float eps, const int32_t* __restrict__ pos_dev,
    int pos_host, int max_len, const RopeTab& rt, uint16_t* __restrict__ k_cache,
    uint16_t* __restrict__ v_cache, int64_t head_stride, float scale,
    float* __restrict__ part, int gsplit, u32x4* __restrict__ pend, int n_pend,
    int32_t* __restrict__ status, int max_polls, int32_t* __restrict__ o_status, u32 tag = 0) {
  __shared__ __align__(16) u32 s_q[GQ][HD / 2];  // rotated q pairs
  __shared__ u32 s_knew[HD / 2], s_vnew[HD / 2];
  __shared__ __align__(16) float s_p[GQ][ACH];
  __shared__ float s_red[4][GQ][HD];
  __shared__ float s_stat[GQ][2];
  // kv head g; this workgroup's GQ query heads start at q0 (gsplit workgroups share a
  // kv head, each with GQ of its GQ * gsplit query heads)
  const int g = by / gsplit, t = threadIdx.x;
  const int q0 = g * GQ * gsplit + (by % gsplit) * GQ;
  const bool writer = by % gsplit == 0;  // appends this token's k / v
  const int wave = t >> 6, lane = t & 63;
  // the position from device memory (a captured graph serves every token) or the
  // host; a grid sized for max_len leaves the chunks past it idle
  const int pos = pos_dev ? __builtin_amdgcn_readfirstlane(*pos_dev) : pos_host;
  // pend (n_pend 16-byte units, nullable): the attention output of a launch that hands
  // it to o_proj inside the launch (k_attn_o), and the o_proj output when the MoE router
  // waits for it there, start as the pending pattern; status (nullable) is reset here,
  // before the launch whose router waves may report a wait that gave up
  if (c == 0 && by == 0) {
    for (int i = t; i < n_pend; i += 256) pend[i] = u32x4{~0u, ~0u, ~0u, ~0u};
    if (status && t == 0) *status = I4_OK;
  }
  const int S = pos + 1, c0 = c * ACH;
  if (pos < 0 || pos >= max_len || c0 >= S) return;
  const bool last = c0 + ACH >= S;  // the chunk that holds pos
  const int64_t kv0 = (int64_t)g * head_stride;
  // the projection rows this workgroup rotates come first: wave w takes query
  // heads w and w + 4, and wave 0 of the last chunk this token's key and value
  constexpr int QPW = (GQ + 3) / 4;
  u32 qraw[QPW], qw = *(const u32*)(qn_w + 2 * lane), kraw = 0, kwn = 0, vraw = 0;
  const u32 qoff = (u32)(2 * lane) * 2u, koff = (u32)((nq + g) * HD) * 2u + qoff,
            voff = (u32)((nq + nkv + g) * HD) * 2u + qoff;
  auto qrow = [&](int i) { return (u32)((q0 + min(wave + 4 * i, GQ - 1)) * HD) * 2u + qoff; };
  if constexpr (!POLL) {
#pragma unroll
    for (int i = 0; i < QPW; ++i) qraw[i] = *(const u32*)((const char*)qkv + qrow(i));
    if (last && wave == 0) {
      kraw = *(const u32*)((const char*)qkv + koff);
      vraw = *(const u32*)((const char*)qkv + voff);
    }
  }
  if (last && wave == 0) kwn = *(const u32*)(kn_w + 2 * lane);
  // K: thread t reads dims [32 (t & 3), +32) of position c0 + (t >> 2), rows < pos
  const int j = t >> 2, qp = t & 3;
  const int kr = min(c0 + j, max(pos - 1, 0));
  const uint16_t* krow = k_cache + kv0 + (int64_t)kr * HD + 32 * qp;
  u32x4 kw[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) kw[u] = ldg16(krow + 8 * u);
  // V: thread t reads dims 2 (t & 63), +1 of positions c0 + 16 (t >> 6) + i
  const int d2 = t & 63, ks = t >> 6;
  u32 vv[16];
#pragma unroll
  for (int i = 0; i < 16; ++i)
    vv[i] = *(const u32*)(v_cache + kv0 + (int64_t)min(c0 + 16 * ks + i, max(pos - 1, 0)) * HD +
                          2 * d2);
  if constexpr (POLL) {  // the K / V loads are in flight: now wait for this token's row
    // word of the pair at half-offset o: byte 2 o of the tagged row
    const rsrc_t rq = rsrc(qkv, (u32)((nq + 2 * nkv) * HD) * 4u);
    auto ld = [&](u32 o, u32& d) {
      const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rq, 2u * o, 0, kCoherent);
      const u32 dv = v.x, tv = v.y;
      d = dv;
      return tv != tag;
    };
    bool late = false;
    for (int it = 0;; ++it) {
      bool p = false;
#pragma unroll
      for (int i = 0; i < QPW; ++i) p |= ld(qrow(i), qraw[i]);
      if (last && wave == 0) {
        p |= ld(koff, kraw);
        p |= ld(voff, vraw);
      }
      if (__builtin_amdgcn_ballot_w64(p) == 0) break;
      if (it >= max_polls) {
        late = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
      asm volatile("" ::: "memory");
    }
    if (late) {
#pragma unroll
      for (int i = 0; i < QPW; ++i) qraw[i] = (u32)Half<XT>::QNAN * 0x10001u;
      if (lane == 0 && o_status) *o_status = I4_ERR_HANDOFF;
    }
  }
#pragma unroll
  for (int i = 0; i < QPW; ++i)
    if (wave + 4 * i < GQ) s_q[wave + 4 * i][lane] = head_norm_rope<XT>(qraw[i], qw, eps, pos, rt);
  if (last && wave == 0) {
    const u32 kn = head_norm_rope<XT>(kraw, kwn, eps, pos, rt);
    s_knew[lane] = kn;
    s_vnew[lane] = vraw;
    if (writer) {
      *(u32*)(k_cache + kv0 + (int64_t)pos * HD + 2 * lane) = kn;
      *(u32*)(v_cache + kv0 + (int64_t)pos * HD + 2 * lane) = vraw;
    }
  }
  __syncthreads();
  if (last && c0 + j >= pos) {  // this token's key replaces the row that was loaded
#pragma unroll
    for (int u = 0; u < 4; ++u)
      kw[u] = u32x4{s_knew[16 * qp + 4 * u], s_knew[16 * qp + 4 * u + 1],
                    s_knew[16 * qp + 4 * u + 2], s_knew[16 * qp + 4 * u + 3]};
  }
  float sc[GQ];
#pragma unroll
  for (int h = 0; h < GQ; ++h) {
    float a = 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const u32x4 qv = *(const u32x4*)&s_q[h][16 * qp + 4 * u];
      a = Half<XT>::dot2(kw[u].x, qv.x, a);
      a = Half<XT>::dot2(kw[u].y, qv.y, a);
      a = Half<XT>::dot2(kw[u].z, qv.z, a);
      a = Half<XT>::dot2(kw[u].w, qv.w, a);
    }
    sc[h] = a;
  }
  const bool kvalid = c0 + j < S;
#pragma unroll
  for (int h = 0; h < GQ; ++h) {
    const float v = group_sum<4>(sc[h]);
    if (qp == 0) s_p[h][j] = kvalid ? v * scale : -__builtin_inff();
  }
  __syncthreads();
  // chunk softmax: 32 threads per query head, two positions each
  {
    const int hh = t >> 5, jj = t & 31;
    if (hh < GQ) {
      const float v0 = s_p[hh][jj], v1 = s_p[hh][jj + 32];
      const float m = group_max<32>(fmaxf(v0, v1));  // position c0 < S is always valid
      const float p0 = expf(v0 - m), p1 = expf(v1 - m);
      s_p[hh][jj] = p0;
      s_p[hh][jj + 32] = p1;
      const float l = group_sum<32>(p0 + p1);
      if (jj == 0) {
        s_stat[hh][0] = m;
        s_stat[hh][1] = l;
      }
    }
  }
  __syncthreads();
  float acc[GQ][2];
#pragma unroll
  for (int h = 0; h < GQ; ++h) acc[h][0] = acc[h][1] = 0.f;
#pragma unroll
  for (int i4 = 0; i4 < 16; i4 += 4) {
    float4 p4[GQ];
#pragma unroll
    for (int h = 0; h < GQ; ++h) p4[h] = *(const float4*)&s_p[h][16 * ks + i4];  // 0 past S
#pragma unroll
    for (int i = i4; i < i4 + 4; ++i) {
      // this token's value at pos, and in place of the rows past it (weight 0, but a
      // cache row never written may hold a NaN)
      const u32 vw = (last && c0 + 16 * ks + i >= pos) ? s_vnew[d2] : vv[i];
      const float v0 = Half<XT>::to_f32((uint16_t)vw);
      const float v1 = Half<XT>::to_f32((uint16_t)(vw >> 16));
#pragma unroll
      for (int h = 0; h < GQ; ++h) {
        const float p = i == i4 ? p4[h].x : i == i4 + 1 ? p4[h].y : i == i4 + 2 ? p4[h].z : p4[h].w;
        acc[h][0] += p * v0;
        acc[h][1] += p * v1;
      }
    }
  }
#pragma unroll
  for (int h = 0; h < GQ; ++h) {
    s_red[ks][h][2 * d2] = acc[h][0];
    s_red[ks][h][2 * d2 + 1] = acc[h][1];
  }
  __syncthreads();
  for (int i = t; i < GQ * HD; i += 256) {
    const int h = i / HD, d = i % HD;
    const float o = (s_red[0][h][d] + s_red[1][h][d]) + (s_red[2][h][d] + s_red[3][h][d]);
    float* dst = part + ((int64_t)c * nq + q0 + h) * PSTR;
    dst[4 + d] = o;
    if (d == 0) {
      dst[0] = s_stat[h][0];
      dst[1] = s_stat[h][1];
    }
  }
}

template <int XT, int GQ>
__global__ __launch_bounds__(256) void k_attn_chunk(
    const uint16_t* __restrict__ qkv, int nq, int nkv, const uint16_t* __restrict__ qn_w,
    const uint16_t* __restrict__ kn_w, float eps, const int32_t* __restrict__ pos_dev,
    int pos_host, int max_len, RopeTab rt, uint16_t* __restrict__ k_cache,
    uint16_t* __restrict__ v_cache, int64_t head_stride, float scale,
    float* __restrict__ part, int gsplit, u32x4* __restrict__ pend, int n_pend,
    int32_t* __restrict__ status) {
  chunk_body<XT, GQ, false>(blockIdx.x, blockIdx.y, qkv, nq, nkv, qn_w, kn_w, eps, pos_dev,
                            pos_host, max_len, rt, k_cache, v_cache, head_stride, scale, part,
                            gsplit, pend, n_pend, status, 0, nullptr);
}

// The hand-over tag of a q|k|v row written while the epoch word holds e: odd, so a
// zero-filled buffer never carries one, and spread over the 32 bits.  The launch after
// the chunks (k_attn_o) advances the epoch, so every call, a replayed graph's too,
// waits for a tag that no earlier call wrote.
__device__ inline u32 qkv_tag(u32 e) { return (2u * e + 1u) * 0x9E3779B1u; }

// The input RMSNorm + q|k|v projection and the attention chunks in one launch: blocks
// [0, n_proj) are the projection's GEMV rows (gemv_ct_body with the norm, their rows
// written through to qkv as (value pair, tag) words for the later blocks), the later
// blocks the chunk workgroups (chunk c, kv head group by), which issue their K / V
// loads and then poll qkv until their words carry this call's tag.  Only later blocks
// wait, and only for earlier ones, so a launch whose workgroups are dispatched in
// block order completes.
struct QkvProj {
  const uint16_t* h;   // the layer's input row (with y: the previous layer's h2)
  const uint16_t* nw;  // input RMSNorm weight
  float eps;
  const int32_t* packed;
  const void* scale;
  const int32_t* zeros;
  int N, K, gshift, n_proj;
  // nullable: the previous layer's slot outputs [8][K] and routing weights [8]; the input
  // row is then h + sum_k w[k] y[k] (K = 2048), written to h_out by the first workgroup
  const uint16_t* y = nullptr;
  const float* w = nullptr;
  uint16_t* h_out = nullptr;
};

// COMP: the projection rows complete their input first (QkvProj::y, the decode step's
// XCD-local experts); a kernel of its own, so the plain form keeps its registers
template <int XT, int ST, int L, int GQ, bool COMP = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(XT == I4_F16 ? 4 : 3))) void k_qkv_chunk(
    QkvProj pr, u32* qkv, const u32* __restrict__ epoch, int nq, int nkv,
    const uint16_t* __restrict__ qn_w, const uint16_t* __restrict__ kn_w, float eps,
    const int32_t* __restrict__ pos_dev, int pos_host, int max_len, RopeTab rt,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache, int64_t head_stride,
    float scale, float* __restrict__ part, int gsplit, int nch, u32x4* __restrict__ pend,
    int n_pend, int32_t* __restrict__ status, int max_polls, int32_t* __restrict__ o_status) {
  extern __shared__ __align__(16) unsigned char lds[];
  const int b = blockIdx.x;
  const u32 tag = qkv_tag(__builtin_amdgcn_readfirstlane(*epoch));
  if (b < pr.n_proj) {
    if constexpr (COMP)
      gemv_ct_body<XT, ST, L, true, false, true, true, true>(
          b, 0, pr.h, 0, pr.packed, 0, pr.scale, 0, pr.zeros, 0, nullptr, 1, pr.N, pr.K,
          pr.gshift, qkv, XT, nullptr, pr.nw, pr.eps, lds, 0, nullptr, tag, pr.y, pr.w,
          pr.h_out);
    else
      gemv_ct_body<XT, ST, L, true, false, true, true>(
          b, 0, pr.h, 0, pr.packed, 0, pr.scale, 0, pr.zeros, 0, nullptr, 1, pr.N, pr.K,
          pr.gshift, qkv, XT, nullptr, pr.nw, pr.eps, lds, 0, nullptr, tag);
    return;
  }
  const int cb = b - pr.n_proj;
  chunk_body<XT, GQ, true>(cb % nch, cb / nch, (const uint16_t*)qkv, nq, nkv, qn_w, kn_w, eps,
                           pos_dev, pos_host, max_len, rt, k_cache, v_cache, head_stride, scale,
                           part, gsplit, pend, n_pend, status, max_polls, o_status, tag);
}

// One workgroup of HD threads per query head merges its chunks (flash-decoding):
// out = o / L with a running maximum M over the chunks in chunk order,
// L = sum_c l_c e^(m_c - M), o = sum_c acc_c e^(m_c - M).  Every load of a batch of
// CMB_B chunks (their statistics, read alike by all threads, and thread t's
// accumulator value) is issued before any is used, so a context of up to
// 64 CMB_B positions costs one memory round trip.
static constexpr int CMB = 1024;  // chunks per head at most (max_len <= 65536)
// chunks per batch of loads: 32, so the Thinker's context 1024 (1025 positions with the
// token, 17 chunks) is one round trip, not two (decode step 743-747 -> 740 us per token,
// 126 VGPRs in the merge launch)
static constexpr int CMB_B = 32;
// Head h's output dimension t (bits in the activation dtype): the merge of the
// chunks' (m, l, acc) partials.
template <int XT>
__device__ inline uint16_t combine_head(const float* __restrict__ part, int nq, int h, int t,
                                        int pos, int max_len) {
  if (pos < 0 || pos >= max_len) return Half<XT>::QNAN;  // no row to attend: no partials
  const int nch = (pos + ACH) / ACH;
  // raw buffer loads, all issued unconditionally (clamped chunk index): a guarded
  // load would be waited for where its branch joins
  const rsrc_t pr = rsrc(part, (u32)nch * (u32)nq * (u32)PSTR * 4u);
  const u32 vml = (u32)h * PSTR * 4u, vac = vml + (4u + (u32)t) * 4u;
  const u32 cs = (u32)nq * PSTR * 4u;  // bytes between chunks
  float M = -__builtin_inff(), L = 0.f, o = 0.f;
  for (int cb = 0; cb < nch; cb += CMB_B) {
    float m[CMB_B], l[CMB_B], a[CMB_B];
#pragma unroll
    for (int i = 0; i < CMB_B; ++i) {
      const int so = (int)((u32)min(cb + i, nch - 1) * cs);
      const u32 m_b = __builtin_amdgcn_raw_buffer_load_b32(pr, vml, so, 0);
      const u32 l_b = __builtin_amdgcn_raw_buffer_load_b32(pr, vml + 4u, so, 0);
      const u32 a_b = __builtin_amdgcn_raw_buffer_load_b32(pr, vac, so, 0);
      m[i] = cb + i < nch ? __builtin_bit_cast(float, m_b) : -__builtin_inff();
      l[i] = __builtin_bit_cast(float, l_b);
      a[i] = __builtin_bit_cast(float, a_b);
    }
    __builtin_amdgcn_sched_barrier(0);  // every load of the batch in flight before any use
    float mb = M;
#pragma unroll
    for (int i = 0; i < CMB_B; ++i) mb = fmaxf(mb, m[i]);
    const float sc = expf(M - mb);  // M = -inf at first: sc = 0
    L *= sc;
    o *= sc;
#pragma unroll
    for (int i = 0; i < CMB_B; ++i) {
      const float w = expf(m[i] - mb);  // 0 for the chunks past nch
      L = fmaf(l[i], w, L);
      o = fmaf(a[i], w, o);
    }
    M = mb;
  }
  return Half<XT>::from_f32(o / L);
}

template <int XT>
__global__ __launch_bounds__(HD) void k_attn_combine(const float* __restrict__ part, int nq,
                                                     const int32_t* __restrict__ pos_dev,
                                                     int pos_host, int max_len,
                                                     uint16_t* __restrict__ out) {
  const int h = blockIdx.x, t = threadIdx.x;
  const int pos = pos_dev ? __builtin_amdgcn_readfirstlane(*pos_dev) : pos_host;
  out[(int64_t)h * HD + t] = combine_head<XT>(part, nq, h, t, pos, max_len);
}

// The combine and o_proj in one launch: blocks [0, nq) merge one head each and
// write its 128 outputs to att as 16-byte stores written through to memory
// (NaN in canonical form; att holds the pending pattern from the chunk launch);
// the later blocks are the o_proj GEMV rows (gemv_ct_body with POLL: their
// first weight loads go out at once, then they poll att), y = W att + residual.
// Only later blocks wait, and only for earlier ones, so a launch whose
// workgroups are dispatched in block order always completes; a wait that gives
// up after max_polls polls leaves its rows NaN.
// RH (the hidden size, 0 for none): the MoE router of the decoder layer runs
// behind the o_proj workgroups (i4_thinker_layer_decode).  Those then write y
// through to memory (it holds the pending pattern from the chunk launch), and
// the last workgroups, four router waves each (router_wave, one expert row per
// wave), issue their router weight loads, wait for the whole of y, and write the
// logits of RMSNorm(y) and (expert 0's wave) that normalised row.  They also arm
// the experts' activations with the pending pattern for the experts launch; a
// router wait that gives up writes I4_ERR_HANDOFF to status.
struct OProj {
  const int32_t* packed;
  const void* scale;
  const int32_t* zeros;
  int N, K, gshift;
};

struct RFold {
  const uint16_t* wr;  // [E][H] router weight
  const uint16_t* nw;  // [H] post-attention norm weight
  float eps;
  uint16_t* xn;        // [H] normalised row out
  uint16_t* logits;    // [E] logits out
  u32x4* act;          // experts' activations to arm, n_act 16-byte words
  int n_act;
  int32_t* status;
  int E;
  int n_o;  // o_proj workgroups
  uint16_t* y_copy = nullptr;  // nullable: y as the router read it, for a later launch
};

// y is not __restrict__: the router waves poll it, and a restrict pointer would let
// the compiler take their loads out of the wait loop.  epoch (nullable): the q|k|v
// hand-over epoch of k_qkv_chunk, advanced here, after the chunks that read it.
template <int XT, int ST, int L, int RH>
__global__ __launch_bounds__(256) void k_attn_o(const float* __restrict__ part, int nq,
                                                const int32_t* __restrict__ pos_dev, int pos_host,
                                                int max_len, uint16_t* __restrict__ att, OProj o,
                                                const uint16_t* __restrict__ residual,
                                                uint16_t* y, int max_polls, RFold r,
                                                int32_t* __restrict__ o_status,
                                                u32* __restrict__ epoch) {
  extern __shared__ __align__(16) unsigned char lds[];
  const int b = blockIdx.x, t = threadIdx.x;
  if (epoch && (b | t) == 0) {
    const u32 e = *epoch;
    __builtin_amdgcn_raw_buffer_store_b32(e + 1u, rsrc(epoch, 4u), 0u, 0, 0);
  }
  if (b < nq) {
    __shared__ __align__(16) uint16_t s_o[HD];
    if (t < HD) {
      const int pos = pos_dev ? __builtin_amdgcn_readfirstlane(*pos_dev) : pos_host;
      const uint16_t v = combine_head<XT>(part, nq, b, t, pos, max_len);
      const float f = Half<XT>::to_f32(v);
      s_o[t] = f != f ? Half<XT>::QNAN : v;
    }
    __syncthreads();
    if (t < HD / 8) {
      const rsrc_t r = rsrc(att + (int64_t)b * HD, HD * 2u);
      __builtin_amdgcn_raw_buffer_store_b128(((const u32x4*)s_o)[t], r, (u32)t * 16u, 0,
                                             kCoherent);
    }
    return;
  }
  if constexpr (RH != 0) {
    if (b >= nq + r.n_o) {
      const int rb = b - nq - r.n_o, nrb = (int)gridDim.x - nq - r.n_o;
      for (int i = rb * 256 + t; i < r.n_act; i += nrb * 256) r.act[i] = u32x4{~0u, ~0u, ~0u, ~0u};
      const int e = rb * 4 + (t >> 6);  // wave-uniform
      if (e >= r.E) return;
      bool late = false;
      router_wave<XT, true, RH, true>(y, r.wr, e, r.nw, r.eps, r.xn, r.logits, max_polls, &late,
                                      r.y_copy);
      if (late && (t & 63) == 0) *r.status = I4_ERR_HANDOFF;
      return;
    }
    gemv_ct_body<XT, ST, L, false, true, true>(b - nq, 0, att, 0, o.packed, 0, o.scale, 0,
                                               o.zeros, 0, nullptr, 1, o.N, o.K, o.gshift, y, XT,
                                               residual, nullptr, 0.f, lds, max_polls, r.status);
  } else {
    gemv_ct_body<XT, ST, L, false, true>(b - nq, 0, att, 0, o.packed, 0, o.scale, 0, o.zeros, 0,
                                         nullptr, 1, o.N, o.K, o.gshift, y, XT, residual, nullptr,
                                         0.f, lds, max_polls, o_status);
  }
}

namespace {

// workspace: the chunk partials [nch][nq][PSTR] fp32 (then, for the launch with
// o_proj, the attention output [nq][HD] at the next 256-byte boundary)
size_t attn_ws(int nq, int max_len) {
  const size_t nch = ((size_t)max_len + ACH - 1) / ACH;
  return nch * nq * PSTR * sizeof(float);
}
// with o_proj: then (at a 256-byte boundary) a 256-byte slot holding the status word of
// the o_proj wait and (128 bytes in) the q|k|v hand-over epoch, then the attention
// output, which ends the workspace -- the router-fold launch keeps its output y directly
// behind it, one pending span over both
size_t attn_o_status_off(int nq, int max_len) {
  return (attn_ws(nq, max_len) + 255) & ~(size_t)255;
}
// the q|k|v hand-over epoch word, on its own line of the status slot
size_t attn_o_epoch_off(int nq, int max_len) { return attn_o_status_off(nq, max_len) + 128; }
size_t attn_o_att_off(int nq, int max_len) { return attn_o_status_off(nq, max_len) + 256; }
size_t attn_o_ws(int nq, int max_len) {
  return attn_o_att_off(nq, max_len) + (size_t)nq * HD * 2;
}

// o_proj behind the attention (k_attn_o), or none (o == nullptr: k_attn_combine);
// route: the MoE router behind o_proj (y then directly follows the attention output,
// and w.N is the hidden size, 1024 or 2048)
struct OLaunch {
  OProj w;
  int st;  // scale dtype
  const void* residual;
  void* y;
  const RFold* route = nullptr;
  bool reset_status = true;  // with route: the chunk launch clears route->status
  int32_t* status = nullptr;  // without route: the o_proj wait's status, cleared likewise
  // the input RMSNorm + q|k|v projection in the chunk launch (k_qkv_chunk): qkv is then
  // its (value pair, tag) row, N * 4 bytes; proj_st: its weight's scale dtype
  const QkvProj* proj = nullptr;
  int proj_st = 0;
};

template <int XT, int ST>
int launch_attn_o(const float* part, int nq, const int32_t* pos_dev, int pos, int max_len,
                  uint16_t* att, const OLaunch& o, u32* epoch, hipStream_t s) {
  const int C = o.w.K / 32, L = gemv_lanes_per_row(C, o.w.N), rpw = 256 / L;
  const int n_o = (o.w.N + rpw - 1) / rpw;
  RFold r{};
  int rh = 0, n_r = 0;
  if (o.route) {
    r = *o.route;
    r.n_o = n_o;
    rh = o.w.N;
    n_r = (r.E + 3) / 4;
  }
  const dim3 grid(nq + n_o + n_r);
  const size_t lds = (size_t)o.w.K * 2 + (size_t)C * 8;
#define I4_AO_CASE(L_, RH_)                                                                   \
  if (L == L_ && rh == RH_) {                                                                 \
    hipLaunchKernelGGL((k_attn_o<XT, ST, L_, RH_>), grid, dim3(256), lds, s, part, nq,        \
                       pos_dev, pos, max_len, att, o.w, (const uint16_t*)o.residual,          \
                       (uint16_t*)o.y, kHandoffPolls, r, o.status, epoch);                    \
    return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;                           \
  }
  I4_AO_CASE(8, 0) I4_AO_CASE(16, 0) I4_AO_CASE(32, 0) I4_AO_CASE(64, 0)
  I4_AO_CASE(8, 1024) I4_AO_CASE(16, 1024) I4_AO_CASE(32, 1024) I4_AO_CASE(64, 1024)
  I4_AO_CASE(8, 2048) I4_AO_CASE(16, 2048) I4_AO_CASE(32, 2048) I4_AO_CASE(64, 2048)
#undef I4_AO_CASE
  return I4_ERR_SHAPE;
}

template <int XT>
int attn_launch(const void* qkv, int nq, int nkv, const void* qn_w, const void* kn_w, float eps,
                const RopeTab& rt, const int32_t* pos_dev, int pos, void* k_cache,
                void* v_cache, int max_len, void* out, void* ws, hipStream_t s,
                const OLaunch* o = nullptr) {
  const int64_t hs = (int64_t)max_len * HD;
  float* part = (float*)ws;
  // device position: every chunk of max_len is launched, those past pos exit at once
  const int nch = ((pos_dev ? max_len : pos + 1) + ACH - 1) / ACH;
  const int gq = nq / nkv;
  const float scale = 1.0f / sqrtf((float)HD);
  // 8 query heads per kv head run as two workgroups of 4 (shorter score and P V
  // chains per workgroup; both load the chunk's K / V): the Thinker's decode step
  // took 829 instead of 874 us per token at context 1024, four workgroups of 2 849
  const int gsplit = gq == 8 ? 2 : 1;
  const dim3 grid(nch, nkv * gsplit);
  // with o_proj, the attention output (and, with the router, y right behind it) start
  // pending
  const int n_pend = !o ? 0 : (nq * HD + (o->route ? o->w.N : 0)) / 8;
  int32_t* st_reset = !o ? nullptr : o->route ? (o->reset_status ? o->route->status : nullptr)
                                               : o->status;
  // with o_proj: the q|k|v hand-over epoch (k_qkv_chunk reads it, k_attn_o advances it)
  u32* epoch = o ? (u32*)((char*)ws + attn_o_epoch_off(nq, max_len)) : nullptr;
  if (o && o->proj) {  // projection rows first, then the chunks, polling qkv
    const QkvProj& pr = *o->proj;
    const size_t lds = (size_t)pr.K * 2 + (size_t)(pr.K / 32) * 8;
    const dim3 fgrid(pr.n_proj + nch * nkv * gsplit);
    int32_t* pst = o->route ? o->route->status : o->status;
#define I4_QC_CASE(ST_, G_)                                                                   \
  if (o->proj_st == ST_ && gq / gsplit == G_)                                                 \
    hipLaunchKernelGGL(pr.y ? (k_qkv_chunk<XT, ST_, 32, G_, true>)                           \
                            : (k_qkv_chunk<XT, ST_, 32, G_, false>),                          \
                       fgrid, dim3(256), lds, s, pr,                                          \
                       (u32*)qkv, epoch, nq, nkv, (const uint16_t*)qn_w,                      \
                       (const uint16_t*)kn_w,                                                 \
                       eps, pos_dev, pos, max_len, rt, (uint16_t*)k_cache, (uint16_t*)v_cache, \
                       hs, scale, part, gsplit, nch, (u32x4*)out, n_pend, st_reset,           \
                       kHandoffPolls, pst);                                                   \
  else
    I4_QC_CASE(I4_F32, 1) I4_QC_CASE(I4_F32, 2) I4_QC_CASE(I4_F32, 4)
    I4_QC_CASE(I4_F16, 1) I4_QC_CASE(I4_F16, 2) I4_QC_CASE(I4_F16, 4)
    I4_QC_CASE(I4_BF16, 1) I4_QC_CASE(I4_BF16, 2) I4_QC_CASE(I4_BF16, 4) return I4_ERR_SHAPE;
#undef I4_QC_CASE
  } else {
#define I4_AC_CASE(G_)                                                                        \
  if (gq / gsplit == G_)                                                                      \
    hipLaunchKernelGGL((k_attn_chunk<XT, G_>), grid, dim3(256), 0, s, (const uint16_t*)qkv,  \
                       nq, nkv, (const uint16_t*)qn_w, (const uint16_t*)kn_w, eps, pos_dev,   \
                       pos, max_len, rt,                                                      \
                       (uint16_t*)k_cache, (uint16_t*)v_cache, hs, scale, part, gsplit,     \
                       (u32x4*)(o ? out : nullptr), n_pend, st_reset);                      \
  else
    I4_AC_CASE(1) I4_AC_CASE(2) I4_AC_CASE(4) return I4_ERR_SHAPE;
#undef I4_AC_CASE
  }
  if (o) {  // out is the attention output buffer in the workspace
    if (hipGetLastError() != hipSuccess) return I4_ERR_LAUNCH;
    if (o->st == I4_F32)
      return launch_attn_o<XT, I4_F32>(part, nq, pos_dev, pos, max_len, (uint16_t*)out, *o, epoch,
                                       s);
    if (o->st == I4_F16)
      return launch_attn_o<XT, I4_F16>(part, nq, pos_dev, pos, max_len, (uint16_t*)out, *o, epoch,
                                       s);
    return launch_attn_o<XT, I4_BF16>(part, nq, pos_dev, pos, max_len, (uint16_t*)out, *o, epoch,
                                      s);
  }
  hipLaunchKernelGGL(k_attn_combine<XT>, dim3(nq), dim3(HD), 0, s, part, nq, pos_dev, pos,
                     max_len, (uint16_t*)out);
  return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;
}

}  // namespace

inline size_t al256(size_t b) { return (b + 255) & ~(size_t)255; }

namespace {

// the q|k|v row of a decode token: N = (nq + 2 nkv) HD values, as (value pair, tag)
// words when the projection runs in the chunk launch (k_qkv_chunk), else as halves
size_t qkv_row_bytes(int nq, int nkv) { return al256((size_t)(nq + 2 * nkv) * HD * 4); }

// workspace of i4_thinker_layer_decode: i4_moe_forward's T = 1 workspace first (so its
// status word sits at i4_moe_status_offset(1, H, I, E, topk)), then the attention's
// (chunk partials, status slot, attention output) with the o_proj output h2 right behind
// it, then the q|k|v row
struct LayerWs {
  size_t part, h2, qkv, bytes;
};
LayerWs layer_ws(int nq, int nkv, int max_len, int H, int I, int E, int topk) {
  LayerWs l;
  l.part = al256(i4_moe_workspace_bytes(1, H, I, E, topk));
  l.h2 = l.part + attn_o_ws(nq, max_len);
  l.qkv = al256(l.h2 + (size_t)H * 2);
  l.bytes = l.qkv + qkv_row_bytes(nq, nkv);
  return l;
}

// The q|k|v projection runs inside the chunk launch (k_qkv_chunk) when it has the GEMV
// shape that launch is built for: 32 lanes per row (the Thinker's 2048 -> 5120) and the
// input norm's one staging round (K <= 4096).
bool qkv_fusable(const i4_qweight& qw) {
  return gemv_lanes_per_row(qw.K / 32, qw.N) == 32 && qw.K <= 4096;
}

}  // namespace
}  // namespace i4

extern "C" {

size_t i4_attn_decode_workspace_bytes(int n_heads, int head_dim, int max_len) {
  if (n_heads < 1 || head_dim != i4::HD || max_len < 1) return 0;
  return i4::attn_ws(n_heads, max_len);
}

size_t i4_attn_decode_o_workspace_bytes(int n_heads, int head_dim, int max_len) {
  if (n_heads < 1 || head_dim != i4::HD || max_len < 1) return 0;
  return i4::attn_o_ws(n_heads, max_len);
}

// the attention entries' checks, made before any launch
static int attn_check(const void* qkv, int x_dtype, int n_heads, int n_kv_heads, int head_dim,
                      const void* q_norm_w, const void* k_norm_w, const float* inv_freq,
                      const int32_t* pos_dev, int pos, void* k_cache, void* v_cache,
                      int max_len, void* out) {
  if (!qkv || !q_norm_w || !k_norm_w || !inv_freq || !k_cache || !v_cache || !out)
    return I4_ERR_NULL;
  if (x_dtype != I4_F16 && x_dtype != I4_BF16) return I4_ERR_DTYPE;
  if (head_dim != i4::HD || n_kv_heads < 1 || n_heads < n_kv_heads || n_heads % n_kv_heads ||
      n_heads / n_kv_heads > i4::GQMAX || n_heads > 1024 || max_len < 1 ||
      max_len > i4::ACH * i4::CMB || (!pos_dev && (pos < 0 || pos >= max_len)))
    return I4_ERR_SHAPE;
  if (((uintptr_t)qkv & 3) || ((uintptr_t)q_norm_w & 3) || ((uintptr_t)k_norm_w & 3) ||
      ((uintptr_t)k_cache & 15) || ((uintptr_t)v_cache & 15) || ((uintptr_t)out & 3) ||
      ((uintptr_t)pos_dev & 3))
    return I4_ERR_ALIGN;
  return I4_OK;
}

static int attn_entry(const void* qkv, int x_dtype, int n_heads, int n_kv_heads, int head_dim,
                      const void* q_norm_w, const void* k_norm_w, float eps,
                      const float* inv_freq, const int32_t* pos_dev, int pos, void* k_cache,
                      void* v_cache, int max_len, void* out, void* workspace,
                      size_t workspace_bytes, hipStream_t stream,
                      const i4::OLaunch* o = nullptr) {
  const int rc = attn_check(qkv, x_dtype, n_heads, n_kv_heads, head_dim, q_norm_w, k_norm_w,
                            inv_freq, pos_dev, pos, k_cache, v_cache, max_len, out);
  if (rc) return rc;
  const size_t need = o ? i4::attn_o_ws(n_heads, max_len) : i4::attn_ws(n_heads, max_len);
  if (!workspace || workspace_bytes < need) return I4_ERR_WORKSPACE;
  if ((uintptr_t)workspace & 255) return I4_ERR_ALIGN;
  i4::RopeTab rt;
  for (int i = 0; i < i4::HD / 2; ++i) rt.inv_freq[i] = inv_freq[i];
  // with o_proj the attention output lives in the workspace, after the partials and the
  // status slot
  void* att = o ? (char*)workspace + i4::attn_o_att_off(n_heads, max_len) : out;
  return x_dtype == I4_F16
             ? i4::attn_launch<I4_F16>(qkv, n_heads, n_kv_heads, q_norm_w, k_norm_w, eps, rt,
                                       pos_dev, pos, k_cache, v_cache, max_len, att, workspace,
                                       stream, o)
             : i4::attn_launch<I4_BF16>(qkv, n_heads, n_kv_heads, q_norm_w, k_norm_w, eps, rt,
                                        pos_dev, pos, k_cache, v_cache, max_len, att, workspace,
                                        stream, o);
}

int i4_attn_decode(const void* qkv, int x_dtype, int n_heads, int n_kv_heads, int head_dim,
                   const void* q_norm_w, const void* k_norm_w, float eps, const float* inv_freq,
                   int pos, void* k_cache, void* v_cache, int max_len, void* out,
                   void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return attn_entry(qkv, x_dtype, n_heads, n_kv_heads, head_dim, q_norm_w, k_norm_w, eps,
                    inv_freq, nullptr, pos, k_cache, v_cache, max_len, out, workspace,
                    workspace_bytes, stream);
}

int i4_attn_decode_at(const void* qkv, int x_dtype, int n_heads, int n_kv_heads, int head_dim,
                      const void* q_norm_w, const void* k_norm_w, float eps,
                      const float* inv_freq, const int32_t* pos, void* k_cache, void* v_cache,
                      int max_len, void* out, void* workspace, size_t workspace_bytes,
                      hipStream_t stream) {
  if (!pos) return I4_ERR_NULL;
  return attn_entry(qkv, x_dtype, n_heads, n_kv_heads, head_dim, q_norm_w, k_norm_w, eps,
                    inv_freq, pos, 0, k_cache, v_cache, max_len, out, workspace,
                    workspace_bytes, stream);
}

int i4_attn_decode_o(const void* qkv, int x_dtype, int n_heads, int n_kv_heads, int head_dim,
                     const void* q_norm_w, const void* k_norm_w, float eps,
                     const float* inv_freq, const int32_t* pos_dev, int pos, void* k_cache,
                     void* v_cache, int max_len, const i4_qweight* o_w, const void* residual,
                     void* y, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (!o_w || !y) return I4_ERR_NULL;
  i4_qweight nw;
  const int rc = i4_check_weight(o_w, &nw);
  if (rc) return rc;
  if (nw.layout != I4_LAYOUT_CT) return I4_ERR_LAYOUT;
  // o_proj: one weight, K = the attention output (one staging round of the poll)
  if (nw.E != 1 || nw.K != n_heads * head_dim || nw.K < 256 || nw.K > 8192)
    return I4_ERR_SHAPE;
  if (((uintptr_t)y & 1) || ((uintptr_t)residual & 1)) return I4_ERR_ALIGN;
  i4::OLaunch o;
  o.w = i4::OProj{nw.packed, nw.scale, nw.zeros, nw.N, nw.K, i4_group_shift(nw.group)};
  o.st = nw.scale_dtype;
  o.residual = residual;
  o.y = y;
  if (workspace && !((uintptr_t)workspace & 255) &&
      workspace_bytes >= i4::attn_o_ws(n_heads, max_len))
    o.status = (int32_t*)((char*)workspace + i4::attn_o_status_off(n_heads, max_len));
  return attn_entry(qkv, x_dtype, n_heads, n_kv_heads, head_dim, q_norm_w, k_norm_w, eps,
                    inv_freq, pos_dev, pos, k_cache, v_cache, max_len, y, workspace,
                    workspace_bytes, stream, &o);
}

size_t i4_attn_decode_o_status_offset(int n_heads, int head_dim, int max_len) {
  if (n_heads < 1 || head_dim != i4::HD || max_len < 1) return 0;
  return i4::attn_o_status_off(n_heads, max_len);
}

// i4_attn_decode_qkv_o's workspace: i4_attn_decode_o's, then the q|k|v row
size_t i4_attn_decode_qkv_o_workspace_bytes(int n_heads, int n_kv_heads, int head_dim,
                                            int max_len) {
  if (n_heads < 1 || n_kv_heads < 1 || head_dim != i4::HD || max_len < 1) return 0;
  return i4::al256(i4::attn_o_ws(n_heads, max_len)) + i4::qkv_row_bytes(n_heads, n_kv_heads);
}

int i4_attn_decode_qkv_o(const void* h, int x_dtype, const void* in_norm_w, float eps,
                         const i4_qweight* qkv_w, int n_heads, int n_kv_heads, int head_dim,
                         const void* q_norm_w, const void* k_norm_w, const float* inv_freq,
                         const int32_t* pos_dev, int pos, void* k_cache, void* v_cache,
                         int max_len, const i4_qweight* o_w, void* y, void* workspace,
                         size_t workspace_bytes, hipStream_t stream) {
  if (!h || !in_norm_w || !qkv_w || !o_w || !y) return I4_ERR_NULL;
  if (x_dtype != I4_F16 && x_dtype != I4_BF16) return I4_ERR_DTYPE;
  i4_qweight qw, ow;
  int rc = i4_check_weight(qkv_w, &qw);
  if (rc) return rc;
  rc = i4_check_weight(o_w, &ow);
  if (rc) return rc;
  if (qw.layout != I4_LAYOUT_CT || ow.layout != I4_LAYOUT_CT) return I4_ERR_LAYOUT;
  if (n_heads < 1 || n_kv_heads < 1 || head_dim != i4::HD) return I4_ERR_SHAPE;
  const int H = ow.N;
  if (qw.E != 1 || qw.K != H || qw.N != (n_heads + 2 * n_kv_heads) * i4::HD) return I4_ERR_SHAPE;
  // o_proj: one staging round of the poll (K <= 8192)
  if (ow.E != 1 || ow.K != n_heads * i4::HD || ow.K < 256 || ow.K > 8192) return I4_ERR_SHAPE;
  if (((uintptr_t)h & 15) || ((uintptr_t)in_norm_w & 15) || ((uintptr_t)y & 1))
    return I4_ERR_ALIGN;
  const size_t need = i4_attn_decode_qkv_o_workspace_bytes(n_heads, n_kv_heads, head_dim, max_len);
  if (!workspace || workspace_bytes < need) return I4_ERR_WORKSPACE;
  if ((uintptr_t)workspace & 255) return I4_ERR_ALIGN;
  char* ws = (char*)workspace;
  void* qkv = ws + i4::al256(i4::attn_o_ws(n_heads, max_len));
  rc = attn_check(qkv, x_dtype, n_heads, n_kv_heads, head_dim, q_norm_w, k_norm_w, inv_freq,
                  pos_dev, pos, k_cache, v_cache, max_len, y);
  if (rc) return rc;
  i4::OLaunch o;
  o.w = i4::OProj{ow.packed, ow.scale, ow.zeros, ow.N, ow.K, i4_group_shift(ow.group)};
  o.st = ow.scale_dtype;
  o.residual = h;
  o.y = y;
  o.status = (int32_t*)(ws + i4::attn_o_status_off(n_heads, max_len));
  i4::QkvProj pr;
  if (i4::qkv_fusable(qw)) {
    pr = i4::QkvProj{(const uint16_t*)h, (const uint16_t*)in_norm_w, eps, qw.packed, qw.scale,
                     qw.zeros, qw.N, qw.K, i4_group_shift(qw.group), (qw.N + 7) / 8};
    o.proj = &pr;
    o.proj_st = qw.scale_dtype;
  } else {
    rc = i4_rmsnorm_linear(h, x_dtype, 1, in_norm_w, eps, &qw, nullptr, qkv, x_dtype, stream);
    if (rc) return rc;
  }
  return attn_entry(qkv, x_dtype, n_heads, n_kv_heads, head_dim, q_norm_w, k_norm_w, eps,
                    inv_freq, pos_dev, pos, k_cache, v_cache, max_len, y, workspace,
                    workspace_bytes, stream, &o);
}

size_t i4_thinker_layer_workspace_bytes(int n_heads, int n_kv_heads, int head_dim, int max_len,
                                        int H, int I, int E, int topk) {
  if (n_heads < 1 || n_kv_heads < 1 || head_dim != i4::HD || max_len < 1) return 0;
  // 0 also for an MoE shape outside the single-launch expert kernel
  if ((H != 1024 && H != 2048) || !i4::moe_m1_ct_fits(topk, H, I)) return 0;
  if (i4_moe_workspace_bytes(1, H, I, E, topk) == 0) return 0;
  return i4::layer_ws(n_heads, n_kv_heads, max_len, H, I, E, topk).bytes;
}

size_t i4_thinker_decode_step_workspace_bytes(int n_heads, int n_kv_heads, int head_dim,
                                              int max_len, int H, int I, int E, int topk) {
  const size_t b =
      i4_thinker_layer_workspace_bytes(n_heads, n_kv_heads, head_dim, max_len, H, I, E, topk);
  // + the hidden state between layers, a copy of the attention output and the slot
  // outputs of the XCD-local experts launch
  return b ? b + 2 * i4::al256((size_t)H * 2) + i4::al256((size_t)8 * H * 2) : 0;
}

// One layer's checks (every one made before any launch) and its launches.
struct LayerOk {
  i4_qweight qw, ow;
  i4::MoeDecodeBufs mb;
  i4::LayerWs l;
};

static int layer_check(const i4_thinker_layer& L, int x_dtype, int n_heads, int n_kv_heads,
                       int head_dim, const float* inv_freq, const int32_t* pos_dev, int pos,
                       int max_len, int topk, void* workspace, size_t workspace_bytes,
                       size_t extra, LayerOk* c) {
  if (!L.in_norm_w || !L.q_norm_w || !L.k_norm_w || !L.k_cache || !L.v_cache) return I4_ERR_NULL;
  if (x_dtype != I4_F16 && x_dtype != I4_BF16) return I4_ERR_DTYPE;
  int rc = i4_check_weight(&L.qkv, &c->qw);
  if (rc) return rc;
  rc = i4_check_weight(&L.o, &c->ow);
  if (rc) return rc;
  if (c->qw.layout != I4_LAYOUT_CT || c->ow.layout != I4_LAYOUT_CT) return I4_ERR_LAYOUT;
  if (!workspace) return I4_ERR_WORKSPACE;
  if ((uintptr_t)workspace & 255) return I4_ERR_ALIGN;
  // the MoE block: CT experts of the single-launch kernel, router and norm present
  rc = i4::moe_decode_bufs(&L.moe, x_dtype, topk, workspace, workspace_bytes, &c->mb);
  if (rc) return rc;
  const int H = c->mb.H;
  if (n_heads < 1 || n_kv_heads < 1 || head_dim != i4::HD) return I4_ERR_SHAPE;
  const i4_qweight &qw = c->qw, &ow = c->ow;
  if (qw.E != 1 || qw.K != H || qw.N != (n_heads + 2 * n_kv_heads) * i4::HD) return I4_ERR_SHAPE;
  // o_proj: one staging round of the poll (K <= 8192), N = H
  if (ow.E != 1 || ow.N != H || ow.K != n_heads * i4::HD || ow.K < 256 || ow.K > 8192)
    return I4_ERR_SHAPE;
  if ((uintptr_t)L.in_norm_w & 15) return I4_ERR_ALIGN;
  c->l = i4::layer_ws(n_heads, n_kv_heads, max_len, H, c->mb.I, c->mb.E, topk);
  if (workspace_bytes < c->l.bytes + extra) return I4_ERR_WORKSPACE;
  char* ws = (char*)workspace;
  return attn_check(ws + c->l.qkv, x_dtype, n_heads, n_kv_heads, head_dim, L.q_norm_w,
                    L.k_norm_w, inv_freq, pos_dev, pos, L.k_cache, L.v_cache, max_len,
                    ws + c->l.h2);
}

// h -> out through one layer; reset: the chunk launch clears the status word.  The
// projection runs in the chunk launch where its shape allows (i4::qkv_fusable).
// XCD-local form (decode step): with slot_y the layer's input is completed in the chunk
// launch, h + sum_k slot_w[k] slot_y[k], and written to h_out (the attention's residual);
// with ypart the experts launch is the XCD-local one, its slot outputs to ypart (the next
// layer completes them) instead of out.
static int layer_launch(const i4_thinker_layer& L, const LayerOk& c, int x_dtype,
                        int n_heads, int n_kv_heads, const float* inv_freq,
                        const int32_t* pos_dev, int pos, int max_len, int topk, int renorm,
                        const void* h, bool reset, void* out, void* workspace,
                        hipStream_t stream, const void* slot_y = nullptr,
                        const float* slot_w = nullptr, void* h_out = nullptr,
                        void* ypart = nullptr, void* h2_copy = nullptr) {
  char* ws = (char*)workspace;
  void* qkv = ws + c.l.qkv;
  void* h2 = ws + c.l.h2;
  int rc;
  const bool fused = i4::qkv_fusable(c.qw);
  if (slot_y && (!fused || c.qw.K != 2048)) return I4_ERR_SHAPE;
  i4::QkvProj pr;
  if (fused) {
    const i4_qweight& qw = c.qw;
    pr = i4::QkvProj{(const uint16_t*)h, (const uint16_t*)L.in_norm_w, L.eps, qw.packed,
                     qw.scale, qw.zeros, qw.N, qw.K, i4_group_shift(qw.group), (qw.N + 7) / 8};
    if (slot_y) {
      pr.y = (const uint16_t*)slot_y;
      pr.w = slot_w;
      pr.h_out = (uint16_t*)h_out;
    }
  } else {
    rc = i4_rmsnorm_linear(h, x_dtype, 1, L.in_norm_w, L.eps, &c.qw, nullptr, qkv, x_dtype,
                           stream);
    if (rc) return rc;
  }
  i4::RFold r{(const uint16_t*)L.moe.router_w, (const uint16_t*)L.moe.norm_w,
              L.moe.norm_eps, c.mb.xn, c.mb.logits, c.mb.act, c.mb.n_act, c.mb.status,
              c.mb.E, 0};
  r.y_copy = (uint16_t*)h2_copy;  // the next layer completes its input from it
  i4::OLaunch o;
  if (fused) {
    o.proj = &pr;
    o.proj_st = c.qw.scale_dtype;
  }
  const i4_qweight& ow = c.ow;
  o.w = i4::OProj{ow.packed, ow.scale, ow.zeros, ow.N, ow.K, i4_group_shift(ow.group)};
  o.st = ow.scale_dtype;
  o.residual = slot_y ? h_out : h;
  o.y = h2;
  o.route = &r;
  o.reset_status = reset;
  rc = attn_entry(qkv, x_dtype, n_heads, n_kv_heads, i4::HD, L.q_norm_w, L.k_norm_w, L.eps,
                  inv_freq, pos_dev, pos, L.k_cache, L.v_cache, max_len, h2, ws + c.l.part,
                  c.l.h2 - c.l.part, stream, &o);
  if (rc) return rc;
  if (ypart) return i4::moe_decode_experts_x(c.mb, x_dtype, topk, renorm, ypart, workspace, stream);
  return i4::moe_decode_experts(c.mb, x_dtype, topk, renorm, h2, out, workspace, stream);
}

int i4_thinker_layer_decode(const void* h, int x_dtype, const void* in_norm_w, float eps,
                            const i4_qweight* qkv_w, int n_heads, int n_kv_heads, int head_dim,
                            const void* q_norm_w, const void* k_norm_w, const float* inv_freq,
                            const int32_t* pos_dev, int pos, void* k_cache, void* v_cache,
                            int max_len, const i4_qweight* o_w, const i4_moe_weights* moe,
                            int topk, int renorm, void* out, void* workspace,
                            size_t workspace_bytes, hipStream_t stream) {
  if (!h || !in_norm_w || !qkv_w || !o_w || !moe || !out) return I4_ERR_NULL;
  if (((uintptr_t)h & 15) || ((uintptr_t)out & 15)) return I4_ERR_ALIGN;
  i4_thinker_layer L;
  L.in_norm_w = in_norm_w;
  L.q_norm_w = q_norm_w;
  L.k_norm_w = k_norm_w;
  L.k_cache = k_cache;
  L.v_cache = v_cache;
  L.eps = eps;
  L.qkv = *qkv_w;
  L.o = *o_w;
  L.moe = *moe;
  LayerOk c;
  const int rc = layer_check(L, x_dtype, n_heads, n_kv_heads, head_dim, inv_freq, pos_dev, pos,
                             max_len, topk, workspace, workspace_bytes, 0, &c);
  if (rc) return rc;
  return layer_launch(L, c, x_dtype, n_heads, n_kv_heads, inv_freq, pos_dev, pos, max_len, topk,
                      renorm, h, true, out, workspace, stream);
}

int i4_thinker_decode_step(const void* h, int x_dtype, const i4_thinker_layer* layers,
                           int n_layers, int n_heads, int n_kv_heads, int head_dim,
                           const float* inv_freq, const int32_t* pos_dev, int pos, int max_len,
                           int topk, int renorm, void* out, void* workspace,
                           size_t workspace_bytes, hipStream_t stream) {
  if (!h || !layers || !out) return I4_ERR_NULL;
  if (n_layers < 1) return I4_ERR_SHAPE;
  if (((uintptr_t)h & 15) || ((uintptr_t)out & 15)) return I4_ERR_ALIGN;
  // every layer's checks first (a host pass per layer, repeated before its launches)
  LayerOk c0, c;
  for (int l = 0; l < n_layers; ++l) {
    int rc = layer_check(layers[l], x_dtype, n_heads, n_kv_heads, head_dim, inv_freq, pos_dev,
                         pos, max_len, topk, workspace, workspace_bytes, 0, l ? &c : &c0);
    if (rc) return rc;
    // every layer shares one workspace layout
    if (l && (c.mb.H != c0.mb.H || c.mb.I != c0.mb.I || c.mb.E != c0.mb.E)) return I4_ERR_SHAPE;
  }
  // the hidden state between layers: one buffer serves them all (a layer reads its input
  // in its first three launches and writes its output in the fourth); then the slot outputs
  const size_t hb = i4::al256((size_t)c0.mb.H * 2);
  if (workspace_bytes < c0.l.bytes + 2 * hb + i4::al256((size_t)8 * c0.mb.H * 2))
    return I4_ERR_WORKSPACE;
  void* hbuf = (char*)workspace + c0.l.bytes;
  // the attention output h2 as the MoE router read it (the h2 buffer itself is set
  // pending by the next layer's chunk launch, whose projection rows read this copy)
  void* h2c = (char*)hbuf + hb;
  void* ypart = (char*)h2c + hb;
  // XCD-local experts launches (every slot's gate_up and down on one XCD, 1.2 us faster
  // than the single-block launch) where every layer allows: each layer but the last leaves
  // its slot outputs, and the next layer's chunk launch completes them into its input row
  // before the input norm (the stack's completion arithmetic: the same h bit for bit)
  bool xl = n_layers > 1 && topk <= 8 && c0.mb.H == 2048 &&
            i4::moe_m1x_ct_fits(topk, c0.mb.H, c0.mb.I);
  for (int l = 0; l < n_layers && xl; ++l) {
    int rc = layer_check(layers[l], x_dtype, n_heads, n_kv_heads, head_dim, inv_freq, pos_dev,
                         pos, max_len, topk, workspace, workspace_bytes, 0, &c);
    if (rc) return rc;
    xl = i4::qkv_fusable(c.qw) && c.qw.K == 2048;
  }
  const void* cur = h;
  for (int l = 0; l < n_layers; ++l) {
    const bool last = l == n_layers - 1;
    void* dst = last ? out : hbuf;
    int rc = layer_check(layers[l], x_dtype, n_heads, n_kv_heads, head_dim, inv_freq, pos_dev,
                         pos, max_len, topk, workspace, workspace_bytes, 0, &c);
    if (rc) return rc;
    if (xl) {
      // layer l > 0 completes the previous layer's h2 (the copy its router wrote)
      rc = layer_launch(layers[l], c, x_dtype, n_heads, n_kv_heads, inv_freq, pos_dev, pos,
                        max_len, topk, renorm, l ? h2c : h, l == 0, out, workspace, stream,
                        l ? ypart : nullptr, l ? c.mb.w : nullptr, l ? hbuf : nullptr,
                        last ? nullptr : ypart, last ? nullptr : h2c);
    } else {
      rc = layer_launch(layers[l], c, x_dtype, n_heads, n_kv_heads, inv_freq, pos_dev, pos,
                        max_len, topk, renorm, cur, l == 0, dst, workspace, stream);
    }
    if (rc) return rc;
    cur = dst;
  }
  return I4_OK;
}

}  // extern "C"
