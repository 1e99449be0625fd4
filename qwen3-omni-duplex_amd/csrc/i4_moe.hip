// Fused int4 MoE block for gfx950 (replaces FusedPackedMoE.forward,
// src/duplex/streaming/fused_packed_moe.py:191-263).
//
// Decode (T = 1), four launches:
//   router logits -> top-k -> k_moe_gate_up<direct> -> k_moe_down_m1
// k_moe_gate_up computes gate row n and up row n of one selected expert in
// the same lanes, so silu(g) * u happens in registers and only the half-
// precision activation [topk][I] is written (the reference writes fp32
// [8][1536] and runs split / silu / mul / cast as separate kernels,
// fused_packed_moe.py:255-257).  k_moe_down_m1 gives each workgroup a slice of
// output rows across ALL selected experts, so the routing-weighted combine and
// the residual add happen in LDS in a fixed expert order: no atomics, the
// result is bit-reproducible run to run.
//
// Prefill / chunks (T > 1):
//   router logits -> top-k -> k_group -> k_moe_gate_up<list> ->
//   k_moe_down_list -> k_moe_combine
// k_group sorts the T*topk (token, slot) pairs by expert (stable in token
// order) and cuts each expert's tokens into entries of at most MT tokens, so
// each weight row is streamed once per entry instead of once per token (the
// reference loops over tokens, fused_packed_moe.py:231).
#include "i4_common.h"
#include "i4_launch.h"
#include "i4_topk.h"

namespace i4 {

static constexpr int WG = 256;
static constexpr int MT_LIST = 4;    // tokens per entry in the grouped GEMV path
static constexpr int TCHUNK = 1024;  // tokens handled by one pass of the pipeline
static constexpr size_t kMaxLds = 65536;  // dynamic LDS per workgroup

struct QW {  // device view of one CT weight
  const int32_t* packed;
  const void* scale;
  const int32_t* zeros;
  int64_t pes, ses, zes;
  int gshift, E, N, K;
};

// row n of expert e (both already clamped to valid values)
template <int ST> __device__ inline RowPtr row_ptr(const QW& w, int e, int n) {
  const int C = w.K >> 5, KW = w.K >> 3;
  const int NG = (C + (1 << w.gshift) - 1) >> w.gshift, NZW = (NG + 7) >> 3;
  RowPtr r;
  r.p = w.packed + e * w.pes + (int64_t)n * KW;
  r.s = scale_at<ST>(w.scale, e * w.ses + (int64_t)n * NG);
  r.z = w.zeros ? (const u32*)w.zeros + e * w.zes + (int64_t)n * NZW : kSymZeros;
  return r;
}

// ---------------------------------------------------------------------------
// gate_up + SiLU.  L lanes per row pair (gate row n, up row I + n); a
// workgroup owns WG/L consecutive row pairs of one entry (one expert and up
// to MT of its tokens).
//   GU_SEL:   decode, entry j is slot j of token 0, experts from sel[]
//   GU_ROUTE: decode, every wave ranks the E logits itself (top-k + softmax,
//             bit-identical in every wave) and takes slot j; workgroup
//             (0, 0) writes sel[] / wts[] for the down projection
//   GU_LIST:  grouped entries {expert, first position, count} from k_group
enum { GU_SEL = 0, GU_ROUTE = 1, GU_LIST = 2 };

template <int XT, int ST, int L, int MT, int MODE>
__global__ __launch_bounds__(WG) void k_moe_gate_up(
    const uint16_t* __restrict__ x, int topk, int32_t* __restrict__ sel,
    const uint16_t* __restrict__ logits, int E_r, int renorm, float* __restrict__ wts,
    const int4* __restrict__ entries, const int* __restrict__ n_entries,
    const int32_t* __restrict__ perm, QW w, int I, uint16_t* __restrict__ act) {
  extern __shared__ __align__(16) unsigned char lds[];
  constexpr int RPW = WG / L;
  constexpr int ROUND = 2;
  const int H = w.K, C = H >> 5;
  const int cpl = (C + L - 1) / L;
  u32x4* xs = (u32x4*)lds;
  float2* sums = (float2*)(lds + (size_t)MT * H * 2);

  int pos0 = blockIdx.y, cnt = 1;
  if constexpr (MODE == GU_LIST) {
    if ((int)blockIdx.y >= *n_entries) return;
  }
  // activations first: their loads retire before the weight loads below
  Stager<XT> st(MT, H);
  auto row_of = [&](int t) -> const uint16_t* {
    if constexpr (MODE == GU_LIST) return x + (int64_t)(perm[pos0 + min(t, cnt - 1)] / topk) * H;
    else return x;
  };
  int e;
  if constexpr (MODE == GU_LIST) {
    const int4 en = entries[blockIdx.y];
    e = en.x;
    pos0 = en.y;
    cnt = en.z;
    st.issue(row_of, 0);
  } else if constexpr (MODE == GU_ROUTE) {
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
  const int rl = threadIdx.x / L, cl = threadIdx.x % L;
  const int n = blockIdx.x * RPW + rl;
  const bool rv = n < I;
  const bool ev = (unsigned)e < (unsigned)w.E;
  const int nn = rv ? n : 0, ee = ev ? e : 0;
  const RowPtr rg = row_ptr<ST>(w, ee, nn), ru = row_ptr<ST>(w, ee, I + nn);

  float ag[MT], au[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) ag[t] = au[t] = 0.f;
  Chunk cg[ROUND], cu[ROUND];
  auto load_round = [&](int r0) {
#pragma unroll
    for (int i = 0; i < ROUND; ++i) {
      const int c = min(cl + (r0 + i) * L, C - 1);
      cg[i] = load_chunk<ST>(rg, c, w.gshift);
      cu[i] = load_chunk<ST>(ru, c, w.gshift);
    }
  };
  auto dot_round = [&](int r0) {
#pragma unroll
    for (int i = 0; i < ROUND; ++i) {
      const int c = cl + (r0 + i) * L;
      if (c < C) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          if (t < cnt) {
            const u32x4* xt = xs + (size_t)t * 4 * C;
            const u32x4 x0 = xt[c], x1 = xt[C + c], x2 = xt[2 * C + c], x3 = xt[3 * C + c];
            const float2 sm = sums[t * C + c];
            ag[t] += chunk_dot<XT, ST>(cg[i], x0, x1, x2, x3, sm, c, w.gshift);
            au[t] += chunk_dot<XT, ST>(cu[i], x0, x1, x2, x3, sm, c, w.gshift);
          }
        }
      }
    }
  };
  // round 0 is peeled: a loop-header wait would hold its weight loads behind
  // the activation loads
  load_round(0);
  st.commit(0, xs, sums);
  st.rest(row_of, xs, sums);
  __syncthreads();
  dot_round(0);
  for (int r0 = ROUND; r0 < cpl; r0 += ROUND) {
    load_round(r0);
    dot_round(r0);
  }
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const float g = group_sum<L>(ag[t]);
    const float u = group_sum<L>(au[t]);
    if (rv && cl == 0 && t < cnt)
      act[(int64_t)(pos0 + t) * I + n] =
          Half<XT>::from_f32(ev ? silu(g) * u : __builtin_nanf(""));
  }
}

// ---------------------------------------------------------------------------
// decode down projection + routing-weighted combine + residual (T = 1).
// Lane groups of L lanes; RW output rows per workgroup; the GPR groups of a
// row split the selected experts (j = gi, gi + GPR, ...).  Every weight load
// of a round (all experts of the group x CR chunks) is issued before the
// activations are staged, so one HBM latency covers the whole workgroup.
template <int L> struct DownShape {
  static constexpr int NGR = 256 / L;
  static constexpr int GPR = NGR >= 8 ? NGR / 8 : 1;
  static constexpr int RW = NGR / GPR;
};

template <int XT, int ST, int L, int JMAX>
__global__ __launch_bounds__(WG) void k_moe_down_m1(
    const uint16_t* __restrict__ act, int topk, const int32_t* __restrict__ sel,
    const float* __restrict__ wts, QW w, const uint16_t* __restrict__ residual,
    uint16_t* __restrict__ out) {
  extern __shared__ __align__(16) unsigned char lds[];
  constexpr int GPR = DownShape<L>::GPR, RW = DownShape<L>::RW;
  constexpr int CR = 4;  // chunks per round
  const int I = w.K, H = w.N, C = I >> 5;
  const int cpl = (C + L - 1) / L;
  u32x4* xs = (u32x4*)lds;
  float2* sums = (float2*)(lds + (size_t)topk * I * 2);
  float* red = (float*)(sums + topk * C);  // [topk][RW]

  static_assert(L * RW >= 64, "the expert group must be uniform across a wave");
  __shared__ float s_w[16];  // routing weights, loaded with the first wave of loads
  // unconditional loads (clamped indices): a guarded load would be waited for
  // where its branch joins, before anything else is issued
  const float wv = wts[min((int)threadIdx.x, topk - 1)];
  const int on = blockIdx.x * RW + (int)threadIdx.x;  // output row of the combine threads
  const bool comb = (int)threadIdx.x < RW && on < H;
  const uint16_t res_raw = *(residual ? residual + min(on, H - 1) : act);
  // activations next (all selected rows, contiguous act[j][I])
  Stager<XT> st(topk, I);
  auto row_of = [&](int j) { return act + (int64_t)j * I; };
  st.issue(row_of, 0);
  const int gi = threadIdx.x / L, cl = threadIdx.x % L;
  const int r = gi % RW;
  const int jg = __builtin_amdgcn_readfirstlane(gi / RW);  // wave-uniform: sel[] via s_load
  const int n = blockIdx.x * RW + r;
  const bool rv = n < H;
  const int nn = rv ? n : 0;

  int ej[JMAX];
  RowPtr rp[JMAX];
#pragma unroll
  for (int jj = 0; jj < JMAX; ++jj) {
    const int j = jg + jj * GPR;
    ej[jj] = j < topk ? sel[j] : -1;
    const int ee = (unsigned)ej[jj] < (unsigned)w.E ? ej[jj] : 0;
    rp[jj] = row_ptr<ST>(w, ee, nn);
  }
  float row[JMAX];
#pragma unroll
  for (int jj = 0; jj < JMAX; ++jj) row[jj] = 0.f;
  Chunk ch[JMAX][CR];
  auto load_round = [&](int r0) {
#pragma unroll
    for (int jj = 0; jj < JMAX; ++jj)
#pragma unroll
      for (int i = 0; i < CR; ++i)
        if (i == 0 || (r0 + i) * L < C)  // wave-uniform: skips rounds past the row's end
          ch[jj][i] = load_chunk<ST>(rp[jj], min(cl + (r0 + i) * L, C - 1), w.gshift);
  };
  auto dot_round = [&](int r0) {
#pragma unroll
    for (int jj = 0; jj < JMAX; ++jj) {
      const int j = jg + jj * GPR;
      if (j < topk) {
        const u32x4* xj = xs + (size_t)j * 4 * C;
#pragma unroll
        for (int i = 0; i < CR; ++i) {
          const int c = cl + (r0 + i) * L;
          if (c < C)
            row[jj] += chunk_dot<XT, ST>(ch[jj][i], xj[c], xj[C + c], xj[2 * C + c], xj[3 * C + c],
                                         sums[j * C + c], c, w.gshift);
        }
      }
    }
  };
  // round 0 is peeled: a loop-header wait would hold its weight loads behind
  // the activation loads
  load_round(0);
  st.commit(0, xs, sums);
  st.rest(row_of, xs, sums);
  if ((int)threadIdx.x < topk) s_w[threadIdx.x] = wv;
  __syncthreads();
  dot_round(0);
  for (int r0 = CR; r0 < cpl; r0 += CR) {
    load_round(r0);
    dot_round(r0);
  }
#pragma unroll
  for (int jj = 0; jj < JMAX; ++jj) {
    const int j = jg + jj * GPR;
    const float v = group_sum<L>(row[jj]);
    if (j < topk && cl == 0)
      red[j * RW + r] = (unsigned)ej[jj] < (unsigned)w.E ? v : __builtin_nanf("");
  }
  __syncthreads();
  if (comb) {
    float y = 0.f;
    for (int j = 0; j < topk; ++j) y += s_w[j] * red[j * RW + (int)threadIdx.x];
    out[on] = Half<XT>::from_f32((residual ? Half<XT>::to_f32(res_raw) : 0.f) + y);
  }
}

// ---------------------------------------------------------------------------
// grouped down projection: ys[slot][n] (fp32) for the tokens of one entry
template <int XT, int ST, int L, int MT>
__global__ __launch_bounds__(WG) void k_moe_down_list(
    const uint16_t* __restrict__ act, const int4* __restrict__ entries,
    const int* __restrict__ n_entries, const int32_t* __restrict__ perm, QW w,
    float* __restrict__ ys) {
  extern __shared__ __align__(16) unsigned char lds[];
  constexpr int RPW = WG / L;
  constexpr int ROUND = 4;
  const int I = w.K, H = w.N, C = I >> 5;
  const int cpl = (C + L - 1) / L;
  u32x4* xs = (u32x4*)lds;
  float2* sums = (float2*)(lds + (size_t)MT * I * 2);
  if ((int)blockIdx.y >= *n_entries) return;
  const int4 en = entries[blockIdx.y];
  const int e = en.x, pos0 = en.y, cnt = en.z;
  Stager<XT> st(MT, I);
  auto row_of = [&](int t) { return act + (int64_t)(pos0 + min(t, cnt - 1)) * I; };
  st.issue(row_of, 0);
  const int rl = threadIdx.x / L, cl = threadIdx.x % L;
  const int n = blockIdx.x * RPW + rl;
  const bool rv = n < H;
  if ((unsigned)e >= (unsigned)w.E) {
    if (rv && cl == 0)
      for (int t = 0; t < cnt; ++t) ys[(int64_t)perm[pos0 + t] * H + n] = __builtin_nanf("");
    return;
  }
  const RowPtr rp = row_ptr<ST>(w, e, rv ? n : 0);
  float acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = 0.f;
  for (int r0 = 0; r0 < cpl; r0 += ROUND) {
    Chunk ch[ROUND];
#pragma unroll
    for (int i = 0; i < ROUND; ++i) ch[i] = load_chunk<ST>(rp, min(cl + (r0 + i) * L, C - 1), w.gshift);
    if (r0 == 0) {
      st.commit(0, xs, sums);
      st.rest(row_of, xs, sums);
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < ROUND; ++i) {
      const int c = cl + (r0 + i) * L;
      if (c < C) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          if (t < cnt) {
            const u32x4* xt = xs + (size_t)t * 4 * C;
            acc[t] += chunk_dot<XT, ST>(ch[i], xt[c], xt[C + c], xt[2 * C + c], xt[3 * C + c],
                                        sums[t * C + c], c, w.gshift);
          }
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const float y = group_sum<L>(acc[t]);
    if (rv && cl == 0 && t < cnt) ys[(int64_t)perm[pos0 + t] * H + n] = y;
  }
}

// out[t][n] = residual[t][n] + sum_j w[t][j] * ys[t*topk + j][n], j ascending
// out[t] = residual[t] + sum_j w[t][j] ys[t][j] in slot order.  KMAX >= topk
// slots are loaded unconditionally (indices clamped) so that all loads of a
// thread are in flight together.
template <int XT, int KMAX>
__global__ __launch_bounds__(WG) void k_moe_combine(const float* __restrict__ ys,
                                                    const float* __restrict__ wts,
                                                    const int32_t* __restrict__ sel, int T,
                                                    int topk, int E, int H,
                                                    const uint16_t* __restrict__ residual,
                                                    uint16_t* __restrict__ out) {
  const int64_t i = min((int64_t)blockIdx.x * WG + threadIdx.x, (int64_t)T * H - 1);
  const int t = (int)(i / H), n = (int)(i - (int64_t)t * H);
  const uint16_t rraw = *(residual ? residual + i : (const uint16_t*)sel);
  int sl[KMAX];
  float wv[KMAX], yv[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    const int s = t * topk + min(j, topk - 1);
    sl[j] = sel[s];
    wv[j] = wts[s];
    yv[j] = ys[(int64_t)s * H + n];
  }
  float y = 0.f;
#pragma unroll
  for (int j = 0; j < KMAX; ++j)
    if (j < topk) y += wv[j] * ((unsigned)sl[j] < (unsigned)E ? yv[j] : __builtin_nanf(""));
  const float r = residual ? Half<XT>::to_f32(rraw) : 0.f;
  if ((int64_t)blockIdx.x * WG + threadIdx.x < (int64_t)T * H) out[i] = Half<XT>::from_f32(r + y);
}

// ---------------------------------------------------------------------------
// MFMA tile path for the grouped experts (T > 1).
//
// One workgroup = up to 64 tokens of one expert (m-blocks of 16) x a column
// tile; wave w owns NB n-blocks of 16 weight rows.  v_mfma_f32_16x16x32_{f16,
// bf16}: lane l supplies A[m = l%16][8 k] and B[8 k][n = l%16] for its
// k-group kb = l/16 and receives D[4 kb + i][l%16], i < 4.  K is walked in
// 128-column superchunks (one quantisation group, G = 128): lane group kb
// loads chunk 4s + kb of its weight row with one 16-byte load, and MFMA step
// t uses word t of that chunk -- a permutation of k that A (the staged
// activations, read in the same order) follows, so the contraction is
// unchanged.
//   fp16: B holds q - z exactly ((M + q) - (M + z), one packed half add per
//         pair), so after the group's 4 steps res += s * D.
//   bf16: B holds M + q exactly (no packed bf16 add on gfx950) and the group
//         correction is res += s * D - s (M + z) S_m with S_m the staged
//         activation sum of token m over the group.
// Every product is exact and accumulation is fp32, as in the GEMV path.
// Activation tiles are double buffered in LDS (token stride 272 B keeps the 16
// tokens of an MFMA on distinct banks), only the m-blocks the entry uses are
// staged, and the next superchunk's weights and activations are loaded while
// the current one is multiplied.
//   GATEUP: NB/2 blocks of gate rows and the same up rows per wave, SiLU in
//           the epilogue, act[pos] in the activation dtype; 32 NB row pairs
//           per workgroup.
//   DOWN:   NB blocks of output rows per wave, ys[slot] in fp32; 64 NB rows
//           per workgroup.
static constexpr int MF_TOK = 64;   // tokens per MFMA entry
static constexpr int MF_SMALL = 16; // experts with at most this many tokens: k_moe_mfma_s
static constexpr int MF_TSTRIDE = 17;  // uint4 per staged token row (16 + 1 pad)
static constexpr int MF_NB = 2;     // n-blocks per wave

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

template <int XT> __device__ inline f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (XT == I4_F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// 8 exact halves M + q of one CT word, in the staged pair order
template <int XT> __device__ inline u32x4 decode8(u32 w) {
  constexpr u32 MK = 0x000F000Fu, MG = Half<XT>::MAGIC2;
  return u32x4{(w & MK) | MG, ((w >> 4) & MK) | MG, ((w >> 8) & MK) | MG, ((w >> 12) & MK) | MG};
}

// fp16 pair (M + q0, M + q1) + nz, nz = (-(M + z), -(M + z)): exactly (q0 - z, q1 - z)
__device__ inline u32 sub_zero(u32 p, u32 nz) {
  return __builtin_bit_cast(u32, __builtin_bit_cast(f16x2, p) + __builtin_bit_cast(f16x2, nz));
}

template <int XT, int ST, bool GATEUP, int NB>
__global__ __launch_bounds__(WG) void k_moe_mfma(
    const uint16_t* __restrict__ src, int topk, const int4* __restrict__ entries,
    const int* __restrict__ n_entries, const int32_t* __restrict__ perm, QW w, int I,
    uint16_t* __restrict__ act, float* __restrict__ ys) {
  constexpr bool EXACT = XT == I4_F16;
  constexpr int COLS = GATEUP ? 32 * NB : 64 * NB;  // row pairs (GATEUP) / rows per workgroup
  static_assert(!GATEUP || NB % 2 == 0, "gate_up pairs gate and up blocks");
  __shared__ u32x4 xs[2][MF_TOK * MF_TSTRIDE];
  __shared__ float xsum[2][MF_TOK];
  if ((int)blockIdx.y >= *n_entries) return;
  const int4 en = entries[blockIdx.y];
  const int e = en.x, pos0 = en.y, cnt = en.z;
  const int K = w.K, SC = K >> 7;  // superchunks
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int ln = lane & 15, kb = lane >> 4;
  const bool ev = (unsigned)e < (unsigned)w.E;
  const int ee = ev ? e : 0;
  const int nmb = (cnt + 15) >> 4;

  // weight rows of this lane (column ln of each n-block)
  RowPtr rp[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    int row;
    if constexpr (GATEUP)
      row = blockIdx.x * COLS + 16 * (NB / 2) * wave + 16 * (nb % (NB / 2)) + ln +
            (nb >= NB / 2 ? I : 0);
    else
      row = blockIdx.x * COLS + 16 * NB * wave + 16 * nb + ln;
    rp[nb] = row_ptr<ST>(w, ee, row);
  }
  // staging role: token tk, chunk kc of the superchunk; wave w stages m-block w
  const int tk = threadIdx.x >> 2, kc = threadIdx.x & 3;
  const bool stager = wave < nmb;  // wave-uniform
  const uint16_t* xrow;
  if constexpr (GATEUP) xrow = src + (int64_t)(perm[pos0 + min(tk, cnt - 1)] / topk) * K;
  else xrow = src + (int64_t)(pos0 + min(tk, cnt - 1)) * K;

  u32x4 xd[4];
  auto issue_x = [&](int sc) {
    if (stager) {
#pragma unroll
      for (int j = 0; j < 4; ++j) xd[j] = ldg16(xrow + 128 * sc + 32 * kc + 8 * j);
    }
  };
  auto commit_x = [&](int buf) {
    if (stager) {
      float sm = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xs[buf][tk * MF_TSTRIDE + kc * 4 + j] = pair_order(xd[j]);
        if constexpr (!EXACT) sm += sum8<XT>(xd[j]).y;
      }
      if constexpr (!EXACT) {
        sm = group_sum<4>(sm);
        if (kc == 0) xsum[buf][tk] = sm;
      }
    }
  };
  Chunk cur[NB], nxt[NB];  // weights of this superchunk / the next one
  auto issue_w = [&](int sc, Chunk* dst) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) dst[nb] = load_chunk<ST>(rp[nb], 4 * sc + kb, w.gshift);
  };

  f32x4 res[4][NB];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) res[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};

  issue_w(0, cur);
  issue_x(0);
  for (int sc = 0; sc < SC; ++sc) {
    const int buf = sc & 1;
    commit_x(buf);
    __syncthreads();
    if (sc + 1 < SC) {
      issue_w(sc + 1, nxt);
      issue_x(sc + 1);
    }
    const int g = (4 * sc + kb) >> w.gshift;
    u32 nz[NB];  // fp16: -(M + z) in both halves
    if constexpr (EXACT) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const u32 z = (cur[nb].z >> (4 * (g & 7))) & 15u;
        nz[nb] = (0xE400u | z) * 0x00010001u;
      }
    }
    f32x4 d[4][NB];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) d[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      u32x4 b[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const u32x4 cw = cur[nb].w;
        b[nb] = decode8<XT>(t == 0 ? cw.x : t == 1 ? cw.y : t == 2 ? cw.z : cw.w);
        if constexpr (EXACT) {
          b[nb].x = sub_zero(b[nb].x, nz[nb]);
          b[nb].y = sub_zero(b[nb].y, nz[nb]);
          b[nb].z = sub_zero(b[nb].z, nz[nb]);
          b[nb].w = sub_zero(b[nb].w, nz[nb]);
        }
      }
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        if (mb < nmb) {
          const u32x4 a = xs[buf][(16 * mb + ln) * MF_TSTRIDE + kb * 4 + t];
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) d[mb][nb] = mfma16<XT>(a, b[nb], d[mb][nb]);
        }
      }
    }
    // per-group correction
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const Chunk& c = cur[nb];
      const float sv = scale_from_raw<ST>(c.s);
      float bv = 0.f;
      if constexpr (!EXACT) bv = -sv * (Half<XT>::MAGIC + (float)((c.z >> (4 * (g & 7))) & 15u));
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        if (mb < nmb) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if constexpr (EXACT)
              res[mb][nb][i] = fmaf(sv, d[mb][nb][i], res[mb][nb][i]);
            else
              res[mb][nb][i] = fmaf(sv, d[mb][nb][i],
                                    fmaf(bv, xsum[buf][16 * mb + 4 * kb + i], res[mb][nb][i]));
          }
        }
      }
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) cur[nb] = nxt[nb];
  }
  // epilogue: lane holds rows m = 16 mb + 4 kb + i of column ln
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 16 * mb + 4 * kb + i;
      if (m < cnt) {
        if constexpr (GATEUP) {
#pragma unroll
          for (int nb = 0; nb < NB / 2; ++nb) {
            const int n = blockIdx.x * COLS + 16 * (NB / 2) * wave + 16 * nb + ln;
            const float v =
                ev ? silu(res[mb][nb][i]) * res[mb][nb + NB / 2][i] : __builtin_nanf("");
            act[(int64_t)(pos0 + m) * I + n] = Half<XT>::from_f32(v);
          }
        } else {
          const int64_t o = (int64_t)perm[pos0 + m] * w.N + blockIdx.x * COLS + 16 * NB * wave + ln;
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) ys[o + 16 * nb] = ev ? res[mb][nb][i] : __builtin_nanf("");
        }
      }
    }
  }
}

// Small entries (<= 16 tokens: one m-block) take k_moe_mfma_s: the same
// contraction and corrections, but each lane loads its own A words straight
// from global memory (16 bytes per MFMA step, the 4 waves of a workgroup hit
// the same L1 lines), so there is no LDS staging and no barrier, and the
// weights and activations of the next two superchunks are in flight while one
// is multiplied (a three-slot register ring, unrolled so every slot index is
// static).
template <int XT, int ST, int NB> struct MfSlot {
  Chunk w[NB];
  u32x4 a[4];
};

template <int XT, int ST, bool GATEUP, int NB>
__global__ __launch_bounds__(WG) void k_moe_mfma_s(
    const uint16_t* __restrict__ src, int topk, const int4* __restrict__ entries,
    const int* __restrict__ n_entries, const int32_t* __restrict__ perm, QW w, int I,
    uint16_t* __restrict__ act, float* __restrict__ ys) {
  constexpr bool EXACT = XT == I4_F16;
  constexpr int COLS = GATEUP ? 32 * NB : 64 * NB;
  static_assert(!GATEUP || NB % 2 == 0, "gate_up pairs gate and up blocks");
  if ((int)blockIdx.y >= *n_entries) return;
  const int4 en = entries[blockIdx.y];
  const int e = en.x, pos0 = en.y, cnt = en.z;
  const int K = w.K, SC = K >> 7;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int ln = lane & 15, kb = lane >> 4;
  const bool ev = (unsigned)e < (unsigned)w.E;
  const int ee = ev ? e : 0;
  RowPtr rp[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    int row;
    if constexpr (GATEUP)
      row = blockIdx.x * COLS + 16 * (NB / 2) * wave + 16 * (nb % (NB / 2)) + ln +
            (nb >= NB / 2 ? I : 0);
    else
      row = blockIdx.x * COLS + 16 * NB * wave + 16 * nb + ln;
    rp[nb] = row_ptr<ST>(w, ee, row);
  }
  // A row of this lane: token ln of the entry (clamped; rows >= cnt are not stored)
  const uint16_t* xrow;
  if constexpr (GATEUP) xrow = src + (int64_t)(perm[pos0 + min(ln, cnt - 1)] / topk) * K;
  else xrow = src + (int64_t)(pos0 + min(ln, cnt - 1)) * K;
  xrow += 32 * kb;

  using Slot = MfSlot<XT, ST, NB>;
  // unconditional (past the end it reloads the last superchunk, an L2 hit), so
  // that the number of loads in flight is the same on every path and the
  // waits before each slot's use stay partial
  auto issue = [&](int sc, Slot& sl) {
    sc = min(sc, SC - 1);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) sl.w[nb] = load_chunk<ST>(rp[nb], 4 * sc + kb, w.gshift);
#pragma unroll
    for (int t = 0; t < 4; ++t) sl.a[t] = ldg16(xrow + 128 * sc + 8 * t);
  };
  f32x4 res[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) res[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int sc, const Slot& sl) {
    const int g = (4 * sc + kb) >> w.gshift;
    f32x4 d[NB];
    u32 nz[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      d[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
      nz[nb] = (0xE400u | ((sl.w[nb].z >> (4 * (g & 7))) & 15u)) * 0x00010001u;
    }
    float sm = 0.f;  // bf16: this lane's part of the activation sum of token ln
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const u32x4 a = pair_order(sl.a[t]);
      if constexpr (!EXACT) sm += sum8<XT>(sl.a[t]).y;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const u32x4 cw = sl.w[nb].w;
        u32x4 b = decode8<XT>(t == 0 ? cw.x : t == 1 ? cw.y : t == 2 ? cw.z : cw.w);
        if constexpr (EXACT) {
          b.x = sub_zero(b.x, nz[nb]);
          b.y = sub_zero(b.y, nz[nb]);
          b.z = sub_zero(b.z, nz[nb]);
          b.w = sub_zero(b.w, nz[nb]);
        }
        d[nb] = mfma16<XT>(a, b, d[nb]);
      }
    }
    // S_m for the rows this lane holds (m = 4 kb + i): total over the 4 lane
    // groups of lane m, gathered with bpermute
    float sr[4] = {0.f, 0.f, 0.f, 0.f};
    if constexpr (!EXACT) {
      float tot = sm;
      tot += __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(((lane + 16) & 63) << 2, __builtin_bit_cast(int, sm)));
      tot += __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(((lane + 32) & 63) << 2, __builtin_bit_cast(int, sm)));
      tot += __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(((lane + 48) & 63) << 2, __builtin_bit_cast(int, sm)));
#pragma unroll
      for (int i = 0; i < 4; ++i)
        sr[i] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((4 * kb + i) << 2, __builtin_bit_cast(int, tot)));
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const float sv = scale_from_raw<ST>(sl.w[nb].s);
      float bv = 0.f;
      if constexpr (!EXACT)
        bv = -sv * (Half<XT>::MAGIC + (float)((sl.w[nb].z >> (4 * (g & 7))) & 15u));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (EXACT) res[nb][i] = fmaf(sv, d[nb][i], res[nb][i]);
        else res[nb][i] = fmaf(sv, d[nb][i], fmaf(bv, sr[i], res[nb][i]));
      }
    }
  };
  Slot s0, s1, s2;
  issue(0, s0);
  issue(1, s1);
  issue(2, s2);
  for (int sc = 0; sc < SC; sc += 3) {
    compute(sc, s0);
    issue(sc + 3, s0);
    if (sc + 1 < SC) compute(sc + 1, s1);
    issue(sc + 4, s1);
    if (sc + 2 < SC) compute(sc + 2, s2);
    issue(sc + 5, s2);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = 4 * kb + i;
    if (m < cnt) {
      if constexpr (GATEUP) {
#pragma unroll
        for (int nb = 0; nb < NB / 2; ++nb) {
          const int n = blockIdx.x * COLS + 16 * (NB / 2) * wave + 16 * nb + ln;
          const float v = ev ? silu(res[nb][i]) * res[nb + NB / 2][i] : __builtin_nanf("");
          act[(int64_t)(pos0 + m) * I + n] = Half<XT>::from_f32(v);
        }
      } else {
        const int64_t o = (int64_t)perm[pos0 + m] * w.N + blockIdx.x * COLS + 16 * NB * wave + ln;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) ys[o + 16 * nb] = ev ? res[nb][i] : __builtin_nanf("");
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Sort (token, slot) pairs by expert, stable in token order, and cut them
// into two lists: experts with <= lo_max tokens get entries of <= lo_chunk
// tokens in `entries`, the others entries of <= MF_TOK tokens in
// `mf_entries`.  One workgroup of 1024 threads (E <= 1024):
//   bits[e][w]: bit b set <=> token 32w + b selected expert e
//   pre [e][w]: popcount of bits[e][0..w)
// and thread e owns expert e for the three exclusive prefix sums (tokens,
// first-list entries, second-list entries), done as wave scans plus a scan of
// the wave totals.
__device__ inline int wave_incl_scan(int v) {
  const int lane = __lane_id();
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int u = __shfl_up(v, d, 64);
    if (lane >= d) v += u;
  }
  return v;
}

__global__ __launch_bounds__(1024) void k_group(const int32_t* __restrict__ sel, int T, int topk,
                                                int E, int lo_max, int lo_chunk,
                                                int32_t* __restrict__ perm,
                                                int4* __restrict__ entries,
                                                int* __restrict__ n_entries,
                                                int4* __restrict__ mf_entries,
                                                int* __restrict__ n_mf_entries) {
  extern __shared__ __align__(16) unsigned char lds[];
  __shared__ int s_wsum[16][3];
  const int TW = (T + 31) >> 5;
  u32* bits = (u32*)lds;
  u32* pre = bits + E * TW;
  const int tid = threadIdx.x, nt = blockDim.x, wave = tid >> 6, lane = tid & 63;
  for (int i = tid; i < E * TW; i += nt) bits[i] = 0u;
  __syncthreads();
  for (int s = tid; s < T * topk; s += nt) {
    const int e = sel[s], t = s / topk;
    if ((unsigned)e < (unsigned)E) atomicOr(&bits[e * TW + (t >> 5)], 1u << (t & 31));
  }
  __syncthreads();
  int c = 0;
  if (tid < E) {
    for (int wd = 0; wd < TW; ++wd) {
      pre[tid * TW + wd] = (u32)c;
      c += __popc(bits[tid * TW + wd]);
    }
  }
  const bool big = c > lo_max;
  const int ne = big ? 0 : (c + lo_chunk - 1) / lo_chunk;
  const int nm = big ? (c + MF_TOK - 1) / MF_TOK : 0;
  const int ic = wave_incl_scan(c), ie = wave_incl_scan(ne), im = wave_incl_scan(nm);
  if (lane == 63) {
    s_wsum[wave][0] = ic;
    s_wsum[wave][1] = ie;
    s_wsum[wave][2] = im;
  }
  __syncthreads();
  int bc = 0, be = 0, bm = 0;  // totals of the waves before this one
  for (int v = 0; v < wave; ++v) {
    bc += s_wsum[v][0];
    be += s_wsum[v][1];
    bm += s_wsum[v][2];
  }
  const int off = bc + ic - c, eoff = be + ie - ne, moff = bm + im - nm;
  if (tid == nt - 1) {  // the last thread's inclusive sums are the totals
    *n_entries = be + ie;
    *n_mf_entries = bm + im;
  }
  int* s_off = (int*)(pre + E * TW);  // [E]
  if (tid < E) s_off[tid] = off;
  __syncthreads();
  for (int s = tid; s < T * topk; s += nt) {
    const int e = sel[s], t = s / topk;
    if ((unsigned)e < (unsigned)E) {
      const u32 word = bits[e * TW + (t >> 5)];
      const int below = __popc(word & ((1u << (t & 31)) - 1u));
      perm[s_off[e] + (int)pre[e * TW + (t >> 5)] + below] = s;
    }
  }
  if (tid < E) {
    if (big) {
      for (int q = 0; q < nm; ++q)
        mf_entries[moff + q] = int4{tid, off + q * MF_TOK, min(MF_TOK, c - q * MF_TOK), 0};
    } else {
      for (int q = 0; q < ne; ++q)
        entries[eoff + q] = int4{tid, off + q * lo_chunk, min(lo_chunk, c - q * lo_chunk), 0};
    }
  }
}

}  // namespace i4

// ===========================================================================
// host side
using namespace i4;

namespace {

inline size_t al256(size_t b) { return (b + 255) & ~(size_t)255; }

struct MoeWs {
  void* logits;
  uint16_t* xn;
  int32_t* sel;
  float* w;
  uint16_t* act;
  float* ys;
  int32_t* perm;
  int4* entries;
  int* n_entries;
  int4* mf_entries;
  int* n_mf_entries;
  size_t bytes;
};

MoeWs carve(void* base, int T, int H, int I, int E, int topk) {
  const int Tc = T < TCHUNK ? T : TCHUNK;
  const size_t Tk = (size_t)Tc * topk;
  MoeWs m;
  size_t o = 0;
  auto take = [&](size_t b) {
    void* p = base ? (char*)base + o : nullptr;
    o += al256(b);
    return p;
  };
  m.logits = take((size_t)Tc * E * 2);
  m.xn = (uint16_t*)take((size_t)Tc * H * 2);
  m.sel = (int32_t*)take(Tk * 4);
  m.w = (float*)take(Tk * 4);
  m.act = (uint16_t*)take(Tk * I * 2);
  m.ys = Tc > 1 ? (float*)take(Tk * H * 4) : nullptr;
  m.perm = (int32_t*)take(Tk * 4);
  m.entries = (int4*)take((E + Tk) * sizeof(int4));
  m.n_entries = (int*)take(4);
  m.mf_entries = (int4*)take((E + Tk / MF_TOK + 1) * sizeof(int4));
  m.n_mf_entries = (int*)take(4);
  m.bytes = o;
  return m;
}

// lanes per output row of the down projections (8..64, 3+ chunks per lane
// when the row is long enough)
inline int lanes_per_row(int C) {
  int L = 8;
  while (L * 2 <= C && L < 64) L *= 2;
  while (L > 8 && C < 3 * L) L /= 2;
  return L;
}

QW to_qw(const i4_qweight& w) {
  QW q;
  q.packed = w.packed;
  q.scale = w.scale;
  q.zeros = w.zeros;
  q.pes = w.packed_estride;
  q.ses = w.scale_estride;
  q.zes = w.zeros_estride;
  q.gshift = i4_group_shift(w.group);
  q.E = w.E;
  q.N = w.N;
  q.K = w.K;
  return q;
}

// gate_up lanes: prefer 2 chunks per lane so a decode layer spreads over
// ~3 workgroups per CU (H = 2048: L = 32, 8 row pairs per workgroup)
inline int gate_up_lanes(int C) {
  int L = 8;
  while (L < 64 && C >= 4 * L) L *= 2;
  return L;
}

// decode / grouped gate_up launch.  mode GU_SEL / GU_ROUTE (one token) or
// GU_LIST (n_entries = upper bound on the grouped entries)
struct GateUpArgs {
  int mode, n_entries, topk, E_r, renorm;
  const void* x;
  int32_t* sel;
  const void* logits;
  float* wts;
  const int4* ent;
  const int* nent;
  const int32_t* perm;
  void* act;
};

template <int XT, int ST, int MT, int MODE>
int launch_gate_up_t(int L, dim3 grid, size_t lds, hipStream_t s, const GateUpArgs& a,
                     const QW& w, int I) {
#define I4_GU_CASE(L_)                                                                          \
  if (L == L_) {                                                                                \
    hipLaunchKernelGGL((k_moe_gate_up<XT, ST, L_, MT, MODE>), grid, dim3(WG), lds, s,           \
                       (const uint16_t*)a.x, a.topk, a.sel, (const uint16_t*)a.logits, a.E_r,   \
                       a.renorm, a.wts, a.ent, a.nent, a.perm, w, I, (uint16_t*)a.act);         \
    return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;                             \
  }
  I4_GU_CASE(8) I4_GU_CASE(16) I4_GU_CASE(32) I4_GU_CASE(64)
#undef I4_GU_CASE
  return I4_ERR_SHAPE;
}

template <int XT, int ST>
int launch_gate_up_dt(const GateUpArgs& a, const QW& w, int I, hipStream_t s) {
  const int H = w.K, C = H / 32;
  const int L = gate_up_lanes(C);
  const int rpw = WG / L;
  dim3 grid((I + rpw - 1) / rpw, a.n_entries);
  const int MT = a.mode == GU_LIST ? MT_LIST : 1;
  const size_t lds = (size_t)MT * (H * 2 + C * 8);
  if (lds > kMaxLds) return I4_ERR_SHAPE;
  if (a.mode == GU_SEL) return launch_gate_up_t<XT, ST, 1, GU_SEL>(L, grid, lds, s, a, w, I);
  if (a.mode == GU_ROUTE) return launch_gate_up_t<XT, ST, 1, GU_ROUTE>(L, grid, lds, s, a, w, I);
  return launch_gate_up_t<XT, ST, MT_LIST, GU_LIST>(L, grid, lds, s, a, w, I);
}

template <int XT, int ST>
int launch_down_m1_t(const void* act, int topk, const int32_t* sel, const float* wts,
                     const QW& w, const void* res, void* out, hipStream_t s) {
  const int I = w.K, C = I / 32;
  const int L = lanes_per_row(C);
  const size_t lds_base = (size_t)topk * (I * 2 + C * 8);
#define I4_DN_CASE(L_, J_)                                                                     \
  if (L == L_ && (topk + DownShape<L_>::GPR - 1) / DownShape<L_>::GPR <= J_) {                 \
    constexpr int RW = DownShape<L_>::RW;                                                      \
    const size_t lds = lds_base + (size_t)topk * RW * 4;                                       \
    if (lds > kMaxLds) return I4_ERR_SHAPE;                                                    \
    hipLaunchKernelGGL((k_moe_down_m1<XT, ST, L_, J_>), dim3((w.N + RW - 1) / RW), dim3(WG),   \
                       lds, s, (const uint16_t*)act, topk, sel, wts, w, (const uint16_t*)res,  \
                       (uint16_t*)out);                                                        \
    return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;                            \
  }
  I4_DN_CASE(8, 2) I4_DN_CASE(16, 2) I4_DN_CASE(8, 4) I4_DN_CASE(16, 4) I4_DN_CASE(32, 8)
  I4_DN_CASE(64, 8)
#undef I4_DN_CASE
  return I4_ERR_SHAPE;
}

template <int XT, int ST>
int launch_down_list_t(int max_entries, const void* act, const int4* ent, const int* nent,
                       const int32_t* perm, const QW& w, float* ys, hipStream_t s) {
  const int I = w.K, C = I / 32;
  const int L = lanes_per_row(C);
  const size_t lds = (size_t)MT_LIST * (I * 2 + C * 8);
  if (lds > kMaxLds) return I4_ERR_SHAPE;
  const int rpw = WG / L;
  dim3 grid((w.N + rpw - 1) / rpw, max_entries);
#define I4_DL_CASE(L_)                                                                      \
  if (L == L_) {                                                                            \
    hipLaunchKernelGGL((k_moe_down_list<XT, ST, L_, MT_LIST>), grid, dim3(WG), lds, s,      \
                       (const uint16_t*)act, ent, nent, perm, w, ys);                       \
    return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;                         \
  }
  I4_DL_CASE(8) I4_DL_CASE(16) I4_DL_CASE(32) I4_DL_CASE(64)
#undef I4_DL_CASE
  return I4_ERR_SHAPE;
}

// the three MoE projections dispatched on (activation dtype, scale dtype)
struct MoeOps {
  int (*gate_up)(const GateUpArgs&, const QW&, int, hipStream_t);
  int (*down_m1)(const void*, int, const int32_t*, const float*, const QW&, const void*, void*,
                 hipStream_t);
  int (*down_list)(int, const void*, const int4*, const int*, const int32_t*, const QW&, float*,
                   hipStream_t);
  int (*mfma_gate_up)(int, const void*, int, const int4*, const int*, const int32_t*, const QW&,
                      int, void*, hipStream_t);
  int (*mfma_down)(int, const void*, const int4*, const int*, const int32_t*, const QW&, float*,
                   hipStream_t);
  int (*mfma_gate_up_s)(int, const void*, int, const int4*, const int*, const int32_t*, const QW&,
                        int, void*, hipStream_t);
  int (*mfma_down_s)(int, const void*, const int4*, const int*, const int32_t*, const QW&, float*,
                     hipStream_t);
};

template <int XT, int ST>
int launch_mfma_gate_up_t(int max_entries, const void* x, int topk, const int4* ent,
                          const int* nent, const int32_t* perm, const QW& w, int I, void* act,
                          hipStream_t s) {
  hipLaunchKernelGGL((k_moe_mfma<XT, ST, true, MF_NB>), dim3(I / (32 * MF_NB), max_entries),
                     dim3(WG), 0, s,
                     (const uint16_t*)x, topk, ent, nent, perm, w, I, (uint16_t*)act,
                     (float*)nullptr);
  return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;
}

template <int XT, int ST>
int launch_mfma_down_t(int max_entries, const void* act, const int4* ent, const int* nent,
                       const int32_t* perm, const QW& w, float* ys, hipStream_t s) {
  hipLaunchKernelGGL((k_moe_mfma<XT, ST, false, MF_NB>), dim3(w.N / (64 * MF_NB), max_entries),
                     dim3(WG), 0, s,
                     (const uint16_t*)act, 0, ent, nent, perm, w, 0, (uint16_t*)nullptr, ys);
  return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;
}

template <int XT, int ST>
int launch_mfma_gate_up_s_t(int max_entries, const void* x, int topk, const int4* ent,
                            const int* nent, const int32_t* perm, const QW& w, int I, void* act,
                            hipStream_t s) {
  hipLaunchKernelGGL((k_moe_mfma_s<XT, ST, true, MF_NB>), dim3(I / (32 * MF_NB), max_entries),
                     dim3(WG), 0, s, (const uint16_t*)x, topk, ent, nent, perm, w, I,
                     (uint16_t*)act, (float*)nullptr);
  return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;
}

template <int XT, int ST>
int launch_mfma_down_s_t(int max_entries, const void* act, const int4* ent, const int* nent,
                         const int32_t* perm, const QW& w, float* ys, hipStream_t s) {
  hipLaunchKernelGGL((k_moe_mfma_s<XT, ST, false, MF_NB>), dim3(w.N / (64 * MF_NB), max_entries),
                     dim3(WG), 0, s, (const uint16_t*)act, 0, ent, nent, perm, w, 0,
                     (uint16_t*)nullptr, ys);
  return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;
}

template <int XT, int ST> constexpr MoeOps moe_ops() {
  return MoeOps{&launch_gate_up_dt<XT, ST>, &launch_down_m1_t<XT, ST>,
                &launch_down_list_t<XT, ST>, &launch_mfma_gate_up_t<XT, ST>,
                &launch_mfma_down_t<XT, ST>, &launch_mfma_gate_up_s_t<XT, ST>,
                &launch_mfma_down_s_t<XT, ST>};
}

bool pick_ops(int xt, int gst, int dst, MoeOps* ops) {
  if (gst != dst) return false;
#define I4_OPS(XT_, ST_)                 \
  if (xt == XT_ && gst == ST_) {         \
    *ops = moe_ops<XT_, ST_>();          \
    return true;                         \
  }
  I4_OPS(I4_F16, I4_F32) I4_OPS(I4_F16, I4_F16) I4_OPS(I4_F16, I4_BF16)
  I4_OPS(I4_BF16, I4_F32) I4_OPS(I4_BF16, I4_F16) I4_OPS(I4_BF16, I4_BF16)
#undef I4_OPS
  return false;
}

int check_moe(const i4_moe_weights* mw, int x_dtype, int T, int topk, i4_qweight* gu,
              i4_qweight* dn) {
  if (!mw) return I4_ERR_NULL;
  int rc = i4_check_weight(&mw->gate_up, gu);
  if (rc) return rc;
  rc = i4_check_weight(&mw->down, dn);
  if (rc) return rc;
  if (gu->layout != I4_LAYOUT_CT || dn->layout != I4_LAYOUT_CT) return I4_ERR_LAYOUT;
  if (x_dtype != I4_F16 && x_dtype != I4_BF16) return I4_ERR_DTYPE;
  const int H = gu->K, I = dn->K, E = gu->E;
  if (gu->N != 2 * I || dn->N != H || dn->E != E) return I4_ERR_SHAPE;
  if (T < 1 || E > 512 || topk < 1 || topk > E || topk > 16) return I4_ERR_SHAPE;
  if (H > 4096 || I > 4096) return I4_ERR_SHAPE;
  return I4_OK;
}

int moe_chunk(const void* x, int xt, int T, const i4_moe_weights* mw, const i4_qweight& gu,
              const i4_qweight& dn, int topk, int renorm, const void* logits, const void* residual,
              void* out, int32_t* sel_out, float* w_out, const MoeWs& ws, hipStream_t s) {
  const int H = gu.K, I = dn.K, E = gu.E;
  MoeOps ops;
  if (!pick_ops(xt, gu.scale_dtype, dn.scale_dtype, &ops)) return I4_ERR_DTYPE;
  int rc;
  int32_t* sel = sel_out ? sel_out : ws.sel;
  float* wts = w_out ? w_out : ws.w;
  const QW qgu = to_qw(gu), qdn = to_qw(dn);
  if (T == 1) {  // decode: router -> gate_up (ranks the logits itself) -> down + combine
    const void* lg = logits;
    if (mw->router_w) {
      rc = i4_launch_router_logits(x, xt, 1, H, mw->router_w, E, mw->norm_w, mw->norm_eps,
                                   mw->norm_w ? ws.xn : nullptr, ws.logits, s);
      if (rc) return rc;
      lg = ws.logits;
      if (mw->norm_w) x = ws.xn;  // the experts run on RMSNorm(x); residual is untouched
    }
    const GateUpArgs a{GU_ROUTE, topk, topk, E, renorm, x, sel, lg, wts,
                       nullptr, nullptr, nullptr, ws.act};
    rc = ops.gate_up(a, qgu, I, s);
    if (rc) return rc;
    return ops.down_m1(ws.act, topk, sel, wts, qdn, residual, out, s);
  }
  const void* lg = logits;
  if (mw->router_w) {
    rc = i4_launch_router_logits(x, xt, T, H, mw->router_w, E, mw->norm_w, mw->norm_eps,
                                 mw->norm_w ? ws.xn : nullptr, ws.logits, s);
    if (rc) return rc;
    lg = ws.logits;
    if (mw->norm_w) x = ws.xn;
  }
  rc = i4_launch_topk(lg, xt, T, E, topk, renorm, sel, wts, nullptr, 0, s);
  if (rc) return rc;
  const int Tk = T * topk;
  const int TW = (T + 31) / 32;
  // G = 128 weights take the MFMA kernels: experts with <= MF_SMALL tokens
  // (one m-block) k_moe_mfma_s, the others k_moe_mfma in entries of <= MF_TOK.
  // Other group sizes take the dot2 GEMV list kernels (entries of <= MT_LIST).
  const bool mfma = gu.group == 128 && dn.group == 128 && I % (32 * MF_NB) == 0 &&
                    H % (64 * MF_NB) == 0;
  const size_t glds = (size_t)2 * E * TW * 4 + (size_t)E * 4;
  hipLaunchKernelGGL(k_group, dim3(1), dim3(1024), glds, s, sel, T, topk, E,
                     mfma ? MF_SMALL : 0x7fffffff, mfma ? MF_SMALL : MT_LIST, ws.perm, ws.entries,
                     ws.n_entries, ws.mf_entries, ws.n_mf_entries);
  if (hipGetLastError() != hipSuccess) return I4_ERR_LAUNCH;
  if (mfma) {
    const int max_s = E < Tk ? E : Tk;                                    // one per expert
    const int max_b = (E < Tk / (MF_SMALL + 1) ? E : Tk / (MF_SMALL + 1)) + Tk / MF_TOK + 1;
    rc = ops.mfma_gate_up_s(max_s, x, topk, ws.entries, ws.n_entries, ws.perm, qgu, I, ws.act, s);
    if (rc) return rc;
    rc = ops.mfma_gate_up(max_b, x, topk, ws.mf_entries, ws.n_mf_entries, ws.perm, qgu, I, ws.act,
                          s);
    if (rc) return rc;
    rc = ops.mfma_down_s(max_s, ws.act, ws.entries, ws.n_entries, ws.perm, qdn, ws.ys, s);
    if (rc) return rc;
    rc = ops.mfma_down(max_b, ws.act, ws.mf_entries, ws.n_mf_entries, ws.perm, qdn, ws.ys, s);
    if (rc) return rc;
  } else {
    const int max_entries = (E < Tk ? E : Tk) + Tk / MT_LIST;
    const GateUpArgs a{GU_LIST, max_entries, topk, E, renorm, x, sel, nullptr, wts,
                       ws.entries, ws.n_entries, ws.perm, ws.act};
    rc = ops.gate_up(a, qgu, I, s);
    if (rc) return rc;
    rc = ops.down_list(max_entries, ws.act, ws.entries, ws.n_entries, ws.perm, qdn, ws.ys, s);
    if (rc) return rc;
  }
  const int64_t tot = (int64_t)T * H;
  dim3 cg((unsigned)((tot + WG - 1) / WG));
#define I4_COMB_CASE(XT_, KM_)                                                                 \
  hipLaunchKernelGGL((k_moe_combine<XT_, KM_>), cg, dim3(WG), 0, s, ws.ys, wts, sel, T, topk, E, \
                     H, (const uint16_t*)residual, (uint16_t*)out)
  if (xt == I4_F16) {
    if (topk <= 8) I4_COMB_CASE(I4_F16, 8);
    else I4_COMB_CASE(I4_F16, 16);
  } else {
    if (topk <= 8) I4_COMB_CASE(I4_BF16, 8);
    else I4_COMB_CASE(I4_BF16, 16);
  }
#undef I4_COMB_CASE
  return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;
}

}  // namespace

extern "C" {

size_t i4_moe_workspace_bytes(int T, int H, int I, int E, int topk) {
  if (T < 1 || H < 1 || I < 1 || E < 1 || topk < 1) return 0;
  return carve(nullptr, T, H, I, E, topk).bytes;
}

int i4_moe_forward(const void* x, int x_dtype, int T, const i4_moe_weights* weights, int topk,
                   int renorm, const void* logits, const void* residual, void* out,
                   int32_t* sel_out, float* w_out, void* workspace, size_t workspace_bytes,
                   hipStream_t stream) {
  i4_qweight gu, dn;
  int rc = check_moe(weights, x_dtype, T, topk, &gu, &dn);
  if (rc) return rc;
  if (!x || !out) return I4_ERR_NULL;
  if (!weights->router_w && !logits) return I4_ERR_NULL;
  if (weights->norm_w && !weights->router_w) return I4_ERR_NULL;
  if ((uintptr_t)weights->norm_w & 15) return I4_ERR_ALIGN;
  if (((uintptr_t)x & 15) || ((uintptr_t)out & 15) || ((uintptr_t)residual & 15))
    return I4_ERR_ALIGN;
  const int H = gu.K, I = dn.K, E = gu.E;
  if (H % 8 || I % 8) return I4_ERR_SHAPE;
  const MoeWs need = carve(nullptr, T, H, I, E, topk);
  if (!workspace || workspace_bytes < need.bytes) return I4_ERR_WORKSPACE;
  if ((uintptr_t)workspace & 255) return I4_ERR_ALIGN;
  const MoeWs ws = carve(workspace, T, H, I, E, topk);
  for (int t0 = 0; t0 < T; t0 += TCHUNK) {
    const int Tc = T - t0 < TCHUNK ? T - t0 : TCHUNK;
    const char* xs = (const char*)x + (size_t)t0 * H * 2;
    const void* lg = logits ? (const char*)logits + (size_t)t0 * E * 2 : nullptr;
    const void* rs = residual ? (const char*)residual + (size_t)t0 * H * 2 : nullptr;
    void* os = (char*)out + (size_t)t0 * H * 2;
    rc = moe_chunk(xs, x_dtype, Tc, weights, gu, dn, topk, renorm, lg, rs, os,
                   sel_out ? sel_out + (size_t)t0 * topk : nullptr,
                   w_out ? w_out + (size_t)t0 * topk : nullptr, ws, stream);
    if (rc) return rc;
  }
  return I4_OK;
}

int i4_moe_gate_up(const void* x, int x_dtype, const i4_qweight* gate_up, const int32_t* sel,
                   int topk, void* act, hipStream_t stream) {
  i4_qweight gu;
  int rc = i4_check_weight(gate_up, &gu);
  if (rc) return rc;
  if (gu.layout != I4_LAYOUT_CT) return I4_ERR_LAYOUT;
  if (!x || !sel || !act) return I4_ERR_NULL;
  if (x_dtype != I4_F16 && x_dtype != I4_BF16) return I4_ERR_DTYPE;
  if (topk < 1 || topk > 65535 || gu.N % 2 || gu.K > 4096) return I4_ERR_SHAPE;
  if (((uintptr_t)x & 15) || ((uintptr_t)act & 15)) return I4_ERR_ALIGN;
  MoeOps ops;
  if (!pick_ops(x_dtype, gu.scale_dtype, gu.scale_dtype, &ops)) return I4_ERR_DTYPE;
  const GateUpArgs a{GU_SEL, topk, topk, 0, 0, x, const_cast<int32_t*>(sel), nullptr, nullptr,
                     nullptr, nullptr, nullptr, act};
  return ops.gate_up(a, to_qw(gu), gu.N / 2, stream);
}

int i4_moe_route_gate_up(const void* x, int x_dtype, const i4_qweight* gate_up,
                         const void* logits, int E_r, int topk, int renorm, int32_t* sel_out,
                         float* w_out, void* act, hipStream_t stream) {
  i4_qweight gu;
  int rc = i4_check_weight(gate_up, &gu);
  if (rc) return rc;
  if (gu.layout != I4_LAYOUT_CT) return I4_ERR_LAYOUT;
  if (!x || !logits || !sel_out || !w_out || !act) return I4_ERR_NULL;
  if (x_dtype != I4_F16 && x_dtype != I4_BF16) return I4_ERR_DTYPE;
  if (E_r < 1 || E_r > 512 || E_r > gu.E || topk < 1 || topk > E_r || topk > 64 || gu.N % 2 ||
      gu.K > 4096)
    return I4_ERR_SHAPE;
  if (((uintptr_t)x & 15) || ((uintptr_t)act & 15)) return I4_ERR_ALIGN;
  MoeOps ops;
  if (!pick_ops(x_dtype, gu.scale_dtype, gu.scale_dtype, &ops)) return I4_ERR_DTYPE;
  const GateUpArgs a{GU_ROUTE, topk, topk, E_r, renorm, x, sel_out, logits, w_out,
                     nullptr, nullptr, nullptr, act};
  return ops.gate_up(a, to_qw(gu), gu.N / 2, stream);
}

int i4_moe_down_combine(const void* act, int x_dtype, const i4_qweight* down, const int32_t* sel,
                        const float* w, int topk, const void* residual, void* out,
                        hipStream_t stream) {
  i4_qweight dn;
  int rc = i4_check_weight(down, &dn);
  if (rc) return rc;
  if (dn.layout != I4_LAYOUT_CT) return I4_ERR_LAYOUT;
  if (!act || !sel || !w || !out) return I4_ERR_NULL;
  if (x_dtype != I4_F16 && x_dtype != I4_BF16) return I4_ERR_DTYPE;
  if (topk < 1 || topk > 16 || dn.K > 4096) return I4_ERR_SHAPE;
  if (((uintptr_t)act & 15) || ((uintptr_t)out & 15) || ((uintptr_t)residual & 15))
    return I4_ERR_ALIGN;
  MoeOps ops;
  if (!pick_ops(x_dtype, dn.scale_dtype, dn.scale_dtype, &ops)) return I4_ERR_DTYPE;
  return ops.down_m1(act, topk, sel, w, to_qw(dn), residual, out, stream);
}

size_t i4_moe_stack_workspace_bytes(int T, int H, int I, int E, int topk) {
  const size_t m = i4_moe_workspace_bytes(T, H, I, E, topk);
  if (!m) return 0;
  return m + al256((size_t)T * H * 2);
}

int i4_moe_stack_forward(const void* x, int x_dtype, int T, const i4_moe_weights* layers,
                         int n_layers, int topk, int renorm, void* out, void* workspace,
                         size_t workspace_bytes, hipStream_t stream) {
  if (!layers || !x || !out) return I4_ERR_NULL;
  if (n_layers < 1) return I4_ERR_SHAPE;
  i4_qweight gu, dn;
  for (int l = 0; l < n_layers; ++l) {
    int rc = check_moe(&layers[l], x_dtype, T, topk, &gu, &dn);
    if (rc) return rc;
    if (!layers[l].router_w) return I4_ERR_NULL;
  }
  int rc = check_moe(&layers[0], x_dtype, T, topk, &gu, &dn);
  const int H = gu.K, I = dn.K, E = gu.E;
  for (int l = 1; l < n_layers; ++l)
    if (layers[l].gate_up.K != H || layers[l].down.K != I || layers[l].gate_up.E != E)
      return I4_ERR_SHAPE;
  const size_t mbytes = i4_moe_workspace_bytes(T, H, I, E, topk);
  if (!workspace || workspace_bytes < mbytes + al256((size_t)T * H * 2)) return I4_ERR_WORKSPACE;
  if ((uintptr_t)workspace & 255) return I4_ERR_ALIGN;
  void* buf = (char*)workspace + mbytes;
  const void* h = x;
  for (int l = 0; l < n_layers; ++l) {
    void* dst = ((n_layers - 1 - l) % 2 == 0) ? out : buf;
    rc = i4_moe_forward(h, x_dtype, T, &layers[l], topk, renorm, nullptr, h, dst, nullptr,
                        nullptr, workspace, mbytes, stream);
    if (rc) return rc;
    h = dst;
  }
  return I4_OK;
}

}  // extern "C"
