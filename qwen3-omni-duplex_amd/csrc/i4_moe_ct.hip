// Decode (T = 1) expert kernels on CT rows (I4_LAYOUT_CT weights), the
// decode path of i4_moe_forward when the block carries CT weights; the tile
// kernels of i4_moe_decode.hip serve blocks that only carry the tile copy.
//
// Rows are read whole: L lanes share one row and each lane loads 16-byte
// chunks along it, so a wavefront streams two to eight full rows (the 1 KB
// rows of the Thinker's gate_up at L = 32).  Decode is latency-bound, and
// these narrow workgroups (8 row pairs of gate_up, 8 output rows of down)
// give the most workgroups per layer.
//   k_ct_gate_up: gate row n and up row I + n of one selected expert in the
//     same lanes, so silu(g) * u happens in registers and only the half-
//     precision activation [topk][I] is written (the reference writes fp32
//     [8][1536] and runs split / silu / mul / cast as separate kernels,
//     fused_packed_moe.py:255-257).
//   k_ct_down_m1: a workgroup owns a slice of output rows across ALL selected
//     experts, so the routing-weighted combine and the residual add happen in
//     LDS in a fixed slot order: no atomics, bit-reproducible run to run.
//   k_ct_moe_m1: both in one launch (the decode path when the block carries
//     its router): the down workgroups issue their weight loads while gate_up
//     streams and take act over from the gate_up workgroups inside the launch.
//     Same arithmetic as the two kernels above, bit for bit.
#include "i4_launch.h"
#include "i4_moe_launch.h"
#include "i4_topk.h"

namespace i4 {

static constexpr int WG = 256;
static constexpr size_t kMaxLds = 65536;  // dynamic LDS per workgroup
enum { GU_SEL = 0, GU_ROUTE = 1 };

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
// workgroup owns WG/L consecutive row pairs of slot blockIdx.y.
//   GU_SEL:   experts from sel[]
//   GU_ROUTE: every wave ranks the E logits itself (top-k + softmax,
//             bit-identical in every wave) and takes its slot; workgroup
//             (0, 0) writes sel[] / wts[] for the down projection

template <int XT, int ST, int L, int MODE, bool HANDOFF, bool XCD_LOCAL = false>
__device__ inline void gate_up_body(int bx, int by, const uint16_t* __restrict__ x, int topk,
                                    int32_t* __restrict__ sel,
                                    const uint16_t* __restrict__ logits, int E_r, int renorm,
                                    float* __restrict__ wts, const QW& w, int I,
                                    uint16_t* __restrict__ act, unsigned char* lds) {
  constexpr int MT = 1;
  constexpr int RPW = WG / L;
  constexpr int ROUND = 2;
  const int H = w.K, C = H >> 5;
  const int cpl = (C + L - 1) / L;
  u32x4* xs = (u32x4*)lds;
  float2* sums = (float2*)(lds + (size_t)MT * H * 2);

  const int pos0 = by, cnt = 1;
  const u32 mg = magic_v<XT>();
  Stager<XT> st(MT, H);
  auto row_of = [&](int) -> const uint16_t* { return x; };
  int e;
  if constexpr (MODE == GU_ROUTE) {
    // the logits are the critical path: load them before the activations
    auto route = [&](auto vpl) -> int {
      constexpr int VPL = decltype(vpl)::value;
      u32 raw[VPL];
      load_row<XT, VPL>(logits, 0, E_r, raw);
      st.issue(row_of, 0);
      if (bx == 0 && by == 0 && threadIdx.x < 64) {
        int my_sel = 0;
        float my_w = 0.f;
        topk_row<XT, VPL>(raw, 0, E_r, topk, renorm, sel, wts, nullptr, 0, &my_sel, &my_w);
        return __builtin_amdgcn_readlane(my_sel, 0);
      }
      return topk_slot<XT, VPL>(raw, E_r, by);
    };
    e = E_r <= 128 ? route(std::integral_constant<int, 2>{})
                   : route(std::integral_constant<int, 8>{});
  } else {
    st.issue(row_of, 0);
    e = sel[by];
  }
  const int rl = threadIdx.x / L, cl = threadIdx.x % L;
  const int n = bx * RPW + rl;
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
  // FULL: every chunk of the round lies inside the row for every lane, so the round runs
  // as one basic block without a per-lane test (same products in the same order)
  auto dot_round = [&](int r0, auto full) {
    constexpr bool FULL = decltype(full)::value;
#pragma unroll
    for (int i = 0; i < ROUND; ++i) {
      const int c = cl + (r0 + i) * L;
      if (FULL || c < C) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          if (t < cnt) {
            const u32x4* xt = xs + (size_t)t * 4 * C;
            const u32x4 x0 = xt[c], x1 = xt[C + c], x2 = xt[2 * C + c], x3 = xt[3 * C + c];
            const float2 sm = sums[t * C + c];
            ag[t] += chunk_dot<XT, ST>(cg[i], x0, x1, x2, x3, sm, c, w.gshift, mg);
            au[t] += chunk_dot<XT, ST>(cu[i], x0, x1, x2, x3, sm, c, w.gshift, mg);
          }
        }
      }
    }
  };
  // round 0 is peeled: a loop-header wait would hold its weight loads behind
  // the activation loads
  auto dot_any = [&](int r0) {
    if ((r0 + ROUND) * L <= C) dot_round(r0, std::true_type{});
    else dot_round(r0, std::false_type{});
  };
  load_round(0);
  st.commit(0, xs, sums);
  st.rest(row_of, xs, sums);
  __syncthreads();
  dot_any(0);
  for (int r0 = ROUND; r0 < cpl; r0 += ROUND) {
    load_round(r0);
    dot_any(r0);
  }
  // HANDOFF: the workgroup's RPW activations (one token) are gathered in LDS and go out
  // as whole 16-byte stores written through to memory, NaN in canonical form.
  // Measured on the decode layer: the last of them reach the polling down workgroups
  // about 2 us sooner than one 2-byte store per value.
  __shared__ __align__(16) uint16_t s_act[RPW];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const float g = group_sum<L>(ag[t]);
    const float u = group_sum<L>(au[t]);
    if (rv && cl == 0 && t < cnt) {
      const float v = ev ? silu(g) * u : __builtin_nanf("");
      if constexpr (HANDOFF) s_act[rl] = v != v ? Half<XT>::QNAN : Half<XT>::from_f32(v);
      else act[(int64_t)(pos0 + t) * I + n] = Half<XT>::from_f32(v);
    }
  }
  if constexpr (HANDOFF) {
    static_assert(MT == 1, "one token per handoff workgroup");
    __syncthreads();
    const int n0 = bx * RPW, nv = min(RPW, I - n0);  // this workgroup's rows below I
    uint16_t* dst = act + (int64_t)pos0 * I + n0;
    if (RPW % 8 == 0 && nv == RPW && (I & 7) == 0) {  // 16-byte aligned whole words
      if ((int)threadIdx.x < RPW / 8) {
        const rsrc_t r = rsrc(dst, (u32)RPW * 2u);
        const u32x4 v = ((const u32x4*)s_act)[threadIdx.x];
        // XCD_LOCAL: into this XCD's L2, where the readers on the same XCD find it
        // before a write-through store would be done (which holds the line meanwhile)
        __builtin_amdgcn_raw_buffer_store_b128(v, r, (u32)threadIdx.x * 16u, 0,
                                               XCD_LOCAL ? kL2Only : kCoherent);
      }
    } else if ((int)threadIdx.x < nv) {
      if constexpr (XCD_LOCAL)
        __hip_atomic_store(dst + threadIdx.x, s_act[threadIdx.x], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_WORKGROUP);
      else
        st_coherent(dst + threadIdx.x, s_act[threadIdx.x]);
    }
  }
}

template <int XT, int ST, int L, int MODE>
__global__ __launch_bounds__(WG) void k_ct_gate_up(
    const uint16_t* __restrict__ x, int topk, int32_t* __restrict__ sel,
    const uint16_t* __restrict__ logits, int E_r, int renorm, float* __restrict__ wts, QW w,
    int I, uint16_t* __restrict__ act, int32_t* __restrict__ status) {
  extern __shared__ __align__(16) unsigned char lds[];
  if (status && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *status = I4_OK;
  gate_up_body<XT, ST, L, MODE, false>(blockIdx.x, blockIdx.y, x, topk, sel, logits, E_r, renorm,
                                       wts, w, I, act, lds);
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

// HANDOFF: the experts and routing weights come from the logits (every wave
// ranks them itself, bit-identical to the gate_up workgroups), and act is
// polled as it is written by the gate_up workgroups of the same launch.
template <int XT, int ST, int L, int JMAX, bool HANDOFF>
__device__ inline void down_body(int bx, const uint16_t* __restrict__ act, int topk,
                                 const int32_t* __restrict__ sel, const float* __restrict__ wts,
                                 const uint16_t* __restrict__ logits, int E_r, int renorm,
                                 const QW& w, const uint16_t* __restrict__ residual,
                                 uint16_t* __restrict__ out, unsigned char* lds,
                                 int32_t* __restrict__ status = nullptr, int max_polls = 0) {
  constexpr int GPR = DownShape<L>::GPR, RW = DownShape<L>::RW;
  constexpr int CR = 3;  // chunks per round (FFN 768 at 8 lanes a row: one full round)
  const int I = w.K, H = w.N, C = I >> 5;
  const int cpl = (C + L - 1) / L;
  u32x4* xs = (u32x4*)lds;
  float2* sums = (float2*)(lds + (size_t)topk * I * 2);
  float* red = (float*)(sums + topk * C);  // [topk][RW]

  static_assert(L * RW >= 64, "the expert group must be uniform across a wave");
  __shared__ float s_w[16];  // routing weights, loaded with the first wave of loads
  const int gi = threadIdx.x / L, cl = threadIdx.x % L;
  const int r = gi % RW;
  const int jg = __builtin_amdgcn_readfirstlane(gi / RW);  // wave-uniform: sel[] via s_load
  int my_sel = 0;
  float wv = 0.f;  // lane j < topk of wave 0: slot j's routing weight
  if constexpr (HANDOFF) {
    auto route = [&](auto vpl) {
      constexpr int VPL = decltype(vpl)::value;
      u32 raw[VPL];
      load_row<XT, VPL>(logits, 0, E_r, raw);
      topk_row<XT, VPL>(raw, 0, E_r, topk, renorm, nullptr, nullptr, nullptr, 0, &my_sel, &wv);
    };
    if (E_r <= 128) route(std::integral_constant<int, 2>{});
    else route(std::integral_constant<int, 8>{});
  } else {
    // unconditional loads (clamped indices): a guarded load would be waited
    // for where its branch joins, before anything else is issued
    wv = wts[min((int)threadIdx.x, topk - 1)];
  }
  const int on = bx * RW + (int)threadIdx.x;  // output row of the combine threads
  const bool comb = (int)threadIdx.x < RW && on < H;
  const uint16_t res_raw = *(residual ? residual + min(on, H - 1) : act);
  // activations next (all selected rows, contiguous act[j][I])
  const u32 mg = magic_v<XT>();
  Stager<XT> st(topk, I);
  auto row_of = [&](int j) { return act + (int64_t)j * I; };
  if constexpr (!HANDOFF) st.issue(row_of, 0);
  const int n = bx * RW + r;
  const bool rv = n < H;
  const int nn = rv ? n : 0;

  int ej[JMAX];
  RowPtr rp[JMAX];
#pragma unroll
  for (int jj = 0; jj < JMAX; ++jj) {
    const int j = jg + jj * GPR;
    if constexpr (HANDOFF) ej[jj] = j < topk ? __builtin_amdgcn_readlane(my_sel, j) : -1;
    else ej[jj] = j < topk ? sel[j] : -1;
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
  // FULL: every slot of the wave is selected and every chunk of the round lies inside the
  // row for every lane, so the round runs as one basic block (its LDS reads all go out
  // before the first product); per row the chunks add up in the same order either way
  auto dot_round = [&](int r0, auto full) {
    constexpr bool FULL = decltype(full)::value;
#pragma unroll
    for (int jj = 0; jj < JMAX; ++jj) {
      const int j = jg + jj * GPR;
      if (FULL || j < topk) {
        const u32x4* xj = xs + (size_t)j * 4 * C;
#pragma unroll
        for (int i = 0; i < CR; ++i) {
          const int c = cl + (r0 + i) * L;
          if (FULL || c < C)
            row[jj] += chunk_dot<XT, ST>(ch[jj][i], xj[c], xj[C + c], xj[2 * C + c], xj[3 * C + c],
                                         sums[j * C + c], c, w.gshift, mg);
        }
      }
    }
  };
  auto dot_any = [&](int r0) {
    if (jg + (JMAX - 1) * GPR < topk && (r0 + CR) * L <= C) dot_round(r0, std::true_type{});
    else dot_round(r0, std::false_type{});
  };
  // round 0 is peeled: a loop-header wait would hold its weight loads behind
  // the activation loads
  load_round(0);
  bool late = false;
  if constexpr (HANDOFF) late = poll_rows<XT>(st, act, max_polls);  // one staging round
  st.commit(0, xs, sums);
  if constexpr (!HANDOFF) st.rest(row_of, xs, sums);
  if ((int)threadIdx.x < topk) s_w[threadIdx.x] = wv;
  __syncthreads();
  dot_any(0);
  for (int r0 = CR; r0 < cpl; r0 += CR) {
    load_round(r0);
    dot_any(r0);
  }
#pragma unroll
  for (int jj = 0; jj < JMAX; ++jj) {
    const int j = jg + jj * GPR;
    // each expert's output rounded to the activation dtype before the weighted
    // sum, as the reference's y.to(x.dtype) does (fused_packed_moe.py:262)
    const float v = Half<XT>::to_f32(Half<XT>::from_f32(group_sum<L>(row[jj])));
    if (j < topk && cl == 0)
      red[j * RW + r] = (unsigned)ej[jj] < (unsigned)w.E ? v : __builtin_nanf("");
  }
  __syncthreads();
  if (comb) {
    float y = 0.f;
    for (int j = 0; j < topk; ++j) y = __builtin_fmaf(s_w[j], red[j * RW + (int)threadIdx.x], y);
    if (late) y = __builtin_nanf("");
    out[on] = Half<XT>::from_f32((residual ? Half<XT>::to_f32(res_raw) : 0.f) + y);
  }
  if constexpr (HANDOFF) {
    if (late && threadIdx.x == 0) *status = I4_ERR_HANDOFF;
  }
}

template <int XT, int ST, int L, int JMAX>
__global__ __launch_bounds__(WG) void k_ct_down_m1(
    const uint16_t* __restrict__ act, int topk, const int32_t* __restrict__ sel,
    const float* __restrict__ wts, QW w, const uint16_t* __restrict__ residual,
    uint16_t* __restrict__ out) {
  extern __shared__ __align__(16) unsigned char lds[];
  down_body<XT, ST, L, JMAX, false>(blockIdx.x, act, topk, sel, wts, nullptr, 0, 0, w, residual,
                                    out, lds);
}

// ---------------------------------------------------------------------------
// One launch for the experts of a decode layer: gate_up workgroups first
// (block b < n_gate: slot b / gx, row block b % gx), then the down
// workgroups, which rank the logits, issue their weight loads and then wait
// for the activations by polling them (poll_rows).  Only later blocks wait,
// and only for earlier ones, so a launch whose workgroups are dispatched in
// block order always completes; the down weights stream while gate_up runs,
// and the kernel boundary between the two projections is gone.
struct MoeM1Args {
  const uint16_t* x;
  int topk;
  int32_t* sel;
  const uint16_t* logits;
  int E_r, renorm;
  float* wts;
  QW gu, dn;
  uint16_t* act;
  const uint16_t* residual;
  uint16_t* out;
  int32_t* status;  // I4_ERR_HANDOFF is stored here by a workgroup whose wait gave up
  int gx, n_gate, max_polls;
};

template <int XT, int ST, int LG, int LD, int JMAX>
__global__ __launch_bounds__(WG) void k_ct_moe_m1(MoeM1Args a) {
  extern __shared__ __align__(16) unsigned char lds[];
  const int b = blockIdx.x;
  if (b < a.n_gate)
    gate_up_body<XT, ST, LG, GU_ROUTE, true>(b % a.gx, b / a.gx, a.x, a.topk, a.sel, a.logits,
                                             a.E_r, a.renorm, a.wts, a.gu, a.dn.K, a.act, lds);
  else
    down_body<XT, ST, LD, JMAX, true>(b - a.n_gate, a.act, a.topk, nullptr, nullptr, a.logits,
                                      a.E_r, a.renorm, a.dn, a.residual, a.out, lds, a.status,
                                      a.max_polls);
}

// ---------------------------------------------------------------------------
// XCD-local decode layer (top-8 on 8 XCDs).  Workgroups go round-robin over the
// XCDs (block b on XCD b % 8, the same residue for every partition size that
// divides 8), so slot j takes every block b with b % 8 == j: the gate_up rows of
// expert sel[j] and its whole down projection run on one XCD.  The gate_up
// workgroups store act[j] written through to memory and then once more into their
// L2 (sc0), where the down workgroups of slot j, on the same XCD, find it: their
// polls (loads served past the L1) see a line that L2 holds dirty without the
// round trip to memory (measured on one MI355X: 0.16-0.24 us from store to a
// poll that sees it, against 0.4-0.64 us written through), and each writes its
// rows of the slot's output y[j], rounded to the activation dtype (the
// reference's y.to(x.dtype), fused_packed_moe.py:262).  The routing-weighted sum
// over the slots and the residual are left to the next launch (the next layer's
// router, k_router_m1ws, or k_moe_sum_m1), whose kernel boundary takes the place
// of the cross-XCD hand-over of the activations.  Per expert, the same dot
// products in the same order as k_ct_moe_m1's down workgroups: the layer is
// bit for bit the same.
static constexpr int XCDS = 8;

// Polls one activation row that producers of the same launch write (kPending16
// until then) with loads served past the L1 (sc1): on the producers' XCD such a load
// is served by a line their L2 holds dirty, elsewhere from memory.  Returns true if
// max_polls passes went by without every value.  Thread t reads words t, t + 256, ...
// of the row (st.d[u]), and only those; the barrier of each pass keeps the loads
// inside the loop.  mid() runs once, after the first pass's loads are issued and
// before they are checked: work on data loaded earlier (loads retire in issue order,
// so it waits for those alone) overlaps the first round trip.
template <int XT, class Mid>
__device__ inline bool poll_row_xcd(Stager<XT, 256>& st, const uint16_t* src, int max_polls,
                                    Mid mid) {
  const rsrc_t r = rsrc(src, (u32)st.total * 16u);
  auto issue = [&]() {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int idx = u * 256 + (int)threadIdx.x;
      if (idx < st.total) st.d[u] = ld16_coherent(r, (u32)idx * 16u);
    }
  };
  issue();
  __builtin_amdgcn_sched_barrier(0);  // the loads go out before mid()'s work
  mid();
  for (int it = 0;; ++it) {
    bool pend = false;
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (u * 256 + (int)threadIdx.x < st.total) pend |= has_pending(st.d[u]);
    if (!__syncthreads_or(pend)) return false;
    if (it >= max_polls) return true;
    __builtin_amdgcn_s_sleep(1);
    issue();
  }
}

// Down projection of slot j for output rows [m RWD, (m + 1) RWD): L lanes per row
// (lane l: chunks l, l + L, ... -- the chunk order of down_body), JR rows per lane
// group.  Expert sel[j] is ranked from the logits by every wave.
template <int XT, int ST, int L, int JR>
__device__ inline void down_slot_body(int j, int m, const uint16_t* __restrict__ act,
                                      const uint16_t* __restrict__ logits, int E_r, const QW& w,
                                      uint16_t* __restrict__ ypart, unsigned char* lds,
                                      int32_t* __restrict__ status, int max_polls) {
  constexpr int RP = WG / L, RWD = RP * JR;
  constexpr int CR = 3;  // chunks per round (FFN 768 at 8 lanes a row: one full round)
  const int I = w.K, H = w.N, C = I >> 5;
  const int cpl = (C + L - 1) / L;
  u32x4* xs = (u32x4*)lds;
  float2* sums = (float2*)(lds + (size_t)I * 2);
  // every wave ranks the logits itself (one ranking wave handing the expert to the
  // others through LDS was slower: 13.26 against 12.82 us per stack layer)
  auto route = [&](auto vpl) -> int {
    constexpr int VPL = decltype(vpl)::value;
    u32 raw[VPL];
    load_row<XT, VPL>(logits, 0, E_r, raw);
    return topk_slot<XT, VPL>(raw, E_r, j);
  };
  const int e = E_r <= 128 ? route(std::integral_constant<int, 2>{})
                           : route(std::integral_constant<int, 8>{});
  const bool ev = (unsigned)e < (unsigned)w.E;
  const int ee = ev ? e : 0;
  const int rl = threadIdx.x / L, cl = threadIdx.x % L;
  const u32 mg = magic_v<XT>();
  RowPtr rp[JR];
#pragma unroll
  for (int jr = 0; jr < JR; ++jr) rp[jr] = row_ptr<ST>(w, ee, min(m * RWD + rl + RP * jr, H - 1));
  float row[JR];
#pragma unroll
  for (int jr = 0; jr < JR; ++jr) row[jr] = 0.f;
  Chunk ch[JR][CR];
  auto load_round = [&](int r0) {
#pragma unroll
    for (int jr = 0; jr < JR; ++jr)
#pragma unroll
      for (int i = 0; i < CR; ++i)
        if (i == 0 || (r0 + i) * L < C)  // wave-uniform: skips rounds past the row's end
          ch[jr][i] = load_chunk<ST>(rp[jr], min(cl + (r0 + i) * L, C - 1), w.gshift);
  };
  // A round whose chunks all lie inside the row for every lane (FULL) runs without a
  // per-lane test: one basic block, so the LDS reads of its chunks, shared by the JR rows,
  // all go out before the first product (the guarded form waits on each chunk's reads in
  // turn).  Per row, the chunks add up in the same order either way.
  // A full first round (below) keeps its first chunk of every row spread into decode
  // pairs (XChunk), spread while the activation row is in flight: 12 more VGPRs a
  // chunk, so one chunk of each row, within the four workgroups per CU the launch needs.
  constexpr bool XP = JR <= 2;  // more rows per lane would cost the launch its occupancy
  XChunk xc[XP ? JR : 1];
  const bool full0 = XP && CR * L <= C;
  auto dot_round = [&](int r0, auto full) {
    constexpr bool FULL = decltype(full)::value;
#pragma unroll
    for (int i = 0; i < CR; ++i) {
      const int c = cl + (r0 + i) * L;
      if (FULL || c < C) {
        const u32x4 x0 = xs[c], x1 = xs[C + c], x2 = xs[2 * C + c], x3 = xs[3 * C + c];
        const float2 sm = sums[c];
#pragma unroll
        for (int jr = 0; jr < JR; ++jr)
          row[jr] += XP && FULL && i == 0 && r0 == 0
                         ? xchunk_dot<XT, ST>(xc[XP ? jr : 0], x0, x1, x2, x3, sm, c, w.gshift)
                         : chunk_dot<XT, ST>(ch[jr][i], x0, x1, x2, x3, sm, c, w.gshift, mg);
      }
    }
  };
  // the weight loads go out first; the activation row is polled behind them
  load_round(0);
  Stager<XT> st(1, I);
  const bool late = poll_row_xcd<XT>(st, act + (int64_t)j * I, max_polls, [&]() {
    if constexpr (XP) {
      if (full0) {
#pragma unroll
        for (int jr = 0; jr < JR; ++jr) {
          xc[jr] = expand_chunk<XT>(ch[jr][0], mg);
          pin(xc[jr]);
        }
      }
    }
  });
  st.commit(0, xs, sums);
  __syncthreads();
  if (full0) dot_round(0, std::true_type{});
  else dot_round(0, std::false_type{});
  for (int r0 = CR; r0 < cpl; r0 += CR) {
    load_round(r0);
    if ((r0 + CR) * L <= C) dot_round(r0, std::true_type{});
    else dot_round(r0, std::false_type{});
  }
#pragma unroll
  for (int jr = 0; jr < JR; ++jr) {
    const int n = m * RWD + rl + RP * jr;
    const float v = group_sum<L>(row[jr]);
    if (cl == 0 && n < H)
      ypart[(int64_t)j * H + n] = ev && !late ? Half<XT>::from_f32(v) : Half<XT>::QNAN;
  }
  if (late && threadIdx.x == 0) *status = I4_ERR_HANDOFF;
}

struct MoeM1xArgs {
  const uint16_t* x;  // the experts' input row (RMSNorm(h) when the block has a norm)
  int32_t* sel;       // written by block 0 with wts: the routing of the layer
  float* wts;
  const uint16_t* logits;
  int E_r, renorm;
  QW gu, dn;
  uint16_t* act;    // [8][I], the pending pattern before the launch
  uint16_t* ypart;  // [8][H] slot outputs
  int32_t* status;  // I4_ERR_HANDOFF is stored here by a down workgroup whose wait gave up
  int n_gate, max_polls;
};

template <int XT, int ST, int LG, int LD>
__global__ __launch_bounds__(WG) void k_ct_moe_m1x(MoeM1xArgs a) {
  extern __shared__ __align__(16) unsigned char lds[];
  const int b = blockIdx.x;
  if (b < a.n_gate) {
    gate_up_body<XT, ST, LG, GU_ROUTE, true, true>(b / XCDS, b % XCDS, a.x, XCDS, a.sel, a.logits,
                                             a.E_r, a.renorm, a.wts, a.gu, a.dn.K, a.act, lds);
  } else {
    const int d = b - a.n_gate;
    down_slot_body<XT, ST, LD, LD / 4>(d % XCDS, d / XCDS, a.act, a.logits, a.E_r, a.dn, a.ypart,
                                       lds, a.status, a.max_polls);
  }
}

// ---------------------------------------------------------------------------
// launchers
// gate_up lanes: prefer 2 chunks per lane so a decode layer spreads over
// ~3 workgroups per CU (H = 2048: L = 32, 8 row pairs per workgroup)
inline int gate_up_lanes(int C) {
  int L = 8;
  while (L < 64 && C >= 4 * L) L *= 2;
  return L;
}

// lanes per output row of the down projection (8..64, 3+ chunks per lane
// when the row is long enough)
inline int down_lanes_per_row(int C) {
  int L = 8;
  while (L * 2 <= C && L < 64) L *= 2;
  while (L > 8 && C < 3 * L) L /= 2;
  return L;
}

inline QW to_qw(const TW& t) {
  return QW{t.packed, t.scale, t.zeros, t.pes, t.ses, t.zes, t.gshift, t.E, t.N, t.K};
}

template <int XT, int ST, int MODE>
static int ct_gate_up_t(int L, dim3 grid, size_t lds, hipStream_t s, const GateUpArgs& a,
                        const QW& w, int I) {
#define I4_GU_CASE(L_)                                                                          \
  if (L == L_) {                                                                                \
    hipLaunchKernelGGL((k_ct_gate_up<XT, ST, L_, MODE>), grid, dim3(WG), lds, s,                \
                       (const uint16_t*)a.x, a.topk, a.sel, (const uint16_t*)a.logits, a.E_r,   \
                       a.renorm, a.wts, w, I, (uint16_t*)a.act, a.status);                      \
    return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;                             \
  }
  I4_GU_CASE(8) I4_GU_CASE(16) I4_GU_CASE(32) I4_GU_CASE(64)
#undef I4_GU_CASE
  return I4_ERR_SHAPE;
}

template <int XT, int ST>
int launch_gate_up_ct(const GateUpArgs& a, const TW& tw, int I, hipStream_t s) {
  const QW w = to_qw(tw);
  const int H = w.K, C = H / 32;
  const int L = gate_up_lanes(C);
  const int rpw = WG / L;
  dim3 grid((I + rpw - 1) / rpw, a.n_slots);
  const size_t lds = (size_t)H * 2 + C * 8;
  if (lds > kMaxLds) return I4_ERR_SHAPE;
  return a.route ? ct_gate_up_t<XT, ST, GU_ROUTE>(L, grid, lds, s, a, w, I)
                 : ct_gate_up_t<XT, ST, GU_SEL>(L, grid, lds, s, a, w, I);
}

template <int XT, int ST>
int launch_down_m1_ct(const void* act, int topk, const int32_t* sel, const float* wts,
                      const TW& tw, const void* res, void* out, hipStream_t s) {
  const QW w = to_qw(tw);
  const int I = w.K, C = I / 32;
  const int L = down_lanes_per_row(C);
  const size_t lds_base = (size_t)topk * (I * 2 + C * 8);
#define I4_DN_CASE(L_, J_)                                                                     \
  if (L == L_ && (topk + DownShape<L_>::GPR - 1) / DownShape<L_>::GPR <= J_) {                 \
    constexpr int RW = DownShape<L_>::RW;                                                      \
    const size_t lds = lds_base + (size_t)topk * RW * 4;                                       \
    if (lds > kMaxLds) return I4_ERR_SHAPE;                                                    \
    hipLaunchKernelGGL((k_ct_down_m1<XT, ST, L_, J_>), dim3((w.N + RW - 1) / RW), dim3(WG),    \
                       lds, s, (const uint16_t*)act, topk, sel, wts, w, (const uint16_t*)res,  \
                       (uint16_t*)out);                                                        \
    return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;                            \
  }
  I4_DN_CASE(8, 2) I4_DN_CASE(16, 2) I4_DN_CASE(8, 4) I4_DN_CASE(16, 4) I4_DN_CASE(32, 8)
  I4_DN_CASE(64, 8)
#undef I4_DN_CASE
  return I4_ERR_SHAPE;
}

// The single-launch layer covers the lane shapes of the usual widths (gate_up
// lanes 8..64; down lanes 8 or 16, i.e. I < 1536) with topk <= 8 and the
// activation rows in one staging round of the down workgroups.
bool moe_m1_ct_fits(int topk, int H, int I) {
  const int LD = down_lanes_per_row(I / 32);
  if (topk > 8 || (LD != 8 && LD != 16)) return false;
  if ((int64_t)topk * (I / 8) > 4 * WG) return false;
  const size_t lds_d = (size_t)topk * (I * 2 + (I / 32) * 8) + (size_t)topk * 8 * 4;
  const size_t lds_g = (size_t)H * 2 + (H / 32) * 8;
  return lds_d <= kMaxLds && lds_g <= kMaxLds;
}

template <int XT, int ST>
int launch_moe_m1_ct(const GateUpArgs& ga, const TW* tgu, const TW& tdn, const void* res,
                     void* out, int32_t* status, int max_polls, hipStream_t s) {
  MoeM1Args a;
  a.dn = to_qw(tdn);
  a.gu = tgu ? to_qw(*tgu) : a.dn;  // without gate_up workgroups only its shape is unused
  const int H = a.dn.N, I = a.dn.K;
  if (!status || max_polls < 0) return I4_ERR_NULL;
  if (!moe_m1_ct_fits(ga.topk, H, I)) return I4_ERR_SHAPE;
  const int LG = gate_up_lanes(H / 32), LD = down_lanes_per_row(I / 32);
  a.x = (const uint16_t*)ga.x;
  a.topk = ga.topk;
  a.sel = ga.sel;
  a.logits = (const uint16_t*)ga.logits;
  a.E_r = ga.E_r;
  a.renorm = ga.renorm;
  a.wts = ga.wts;
  a.act = (uint16_t*)ga.act;
  a.residual = (const uint16_t*)res;
  a.out = (uint16_t*)out;
  a.status = status;
  a.max_polls = max_polls;
  const int rpw = WG / LG;
  a.gx = (I + rpw - 1) / rpw;
  a.n_gate = tgu ? a.gx * ga.topk : 0;
  constexpr int RW = 8;  // DownShape<8>::RW == DownShape<16>::RW
  static_assert(DownShape<8>::RW == RW && DownShape<16>::RW == RW, "down rows per workgroup");
  const size_t lds_d = (size_t)ga.topk * (I * 2 + (I / 32) * 8) + (size_t)ga.topk * RW * 4;
  const size_t lds_g = (size_t)H * 2 + (H / 32) * 8;
  const size_t lds = lds_d > lds_g ? lds_d : lds_g;
  const dim3 grid(a.n_gate + (H + RW - 1) / RW);
#define I4_M1_CASE(LG_, LD_, J_)                                                              \
  if (LG == LG_ && LD == LD_) {                                                               \
    hipLaunchKernelGGL((k_ct_moe_m1<XT, ST, LG_, LD_, J_>), grid, dim3(WG), lds, s, a);      \
    return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;                           \
  }
  I4_M1_CASE(8, 8, 2) I4_M1_CASE(16, 8, 2) I4_M1_CASE(32, 8, 2) I4_M1_CASE(64, 8, 2)
  I4_M1_CASE(8, 16, 4) I4_M1_CASE(16, 16, 4) I4_M1_CASE(32, 16, 4) I4_M1_CASE(64, 16, 4)
#undef I4_M1_CASE
  return I4_ERR_SHAPE;
}

// The XCD-local layer covers top-8 blocks with the single-launch kernel's lane
// shapes (down lanes 8 or 16: 64 output rows per down workgroup).
bool moe_m1x_ct_fits(int topk, int H, int I) {
  return topk == XCDS && moe_m1_ct_fits(topk, H, I) && (H % 8) == 0;
}

template <int XT, int ST>
int launch_moe_m1x_ct(const GateUpArgs& ga, const TW& tgu, const TW& tdn, void* ypart,
                      int32_t* status, int max_polls, bool down_only, hipStream_t s) {
  MoeM1xArgs a;
  a.gu = to_qw(tgu);
  a.dn = to_qw(tdn);
  const int H = a.dn.N, I = a.dn.K;
  if (!status || max_polls < 0) return I4_ERR_NULL;
  if (!moe_m1x_ct_fits(ga.topk, H, I)) return I4_ERR_SHAPE;
  const int LG = gate_up_lanes(H / 32), LD = down_lanes_per_row(I / 32);
  a.x = (const uint16_t*)ga.x;
  a.sel = ga.sel;
  a.logits = (const uint16_t*)ga.logits;
  a.E_r = ga.E_r;
  a.renorm = ga.renorm;
  a.wts = ga.wts;
  a.act = (uint16_t*)ga.act;
  a.ypart = (uint16_t*)ypart;
  a.status = status;
  a.max_polls = max_polls;
  const int rpw = WG / LG;
  a.n_gate = down_only ? 0 : ((I + rpw - 1) / rpw) * XCDS;  // 0: the down workgroups alone
  constexpr int RWD = 64;  // (WG / LD) * (LD / 4) output rows per down workgroup
  const int n_down = ((H + RWD - 1) / RWD) * XCDS;
  const size_t lds_d = (size_t)I * 2 + (size_t)(I / 32) * 8;
  const size_t lds_g = (size_t)H * 2 + (H / 32) * 8;
  const size_t lds = lds_d > lds_g ? lds_d : lds_g;
  const dim3 grid(a.n_gate + n_down);
#define I4_M1X_CASE(LG_, LD_)                                                                 \
  if (LG == LG_ && LD == LD_) {                                                               \
    hipLaunchKernelGGL((k_ct_moe_m1x<XT, ST, LG_, LD_>), grid, dim3(WG), lds, s, a);          \
    return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;                           \
  }
  I4_M1X_CASE(8, 8) I4_M1X_CASE(16, 8) I4_M1X_CASE(32, 8) I4_M1X_CASE(64, 8)
  I4_M1X_CASE(8, 16) I4_M1X_CASE(16, 16) I4_M1X_CASE(32, 16) I4_M1X_CASE(64, 16)
#undef I4_M1X_CASE
  return I4_ERR_SHAPE;
}

#define I4_INST(XT_, ST_)                                                                      \
  template int launch_gate_up_ct<XT_, ST_>(const GateUpArgs&, const TW&, int, hipStream_t);    \
  template int launch_down_m1_ct<XT_, ST_>(const void*, int, const int32_t*, const float*,     \
                                           const TW&, const void*, void*, hipStream_t);        \
  template int launch_moe_m1_ct<XT_, ST_>(const GateUpArgs&, const TW*, const TW&, const void*, \
                                          void*, int32_t*, int, hipStream_t);                  \
  template int launch_moe_m1x_ct<XT_, ST_>(const GateUpArgs&, const TW&, const TW&, void*,      \
                                           int32_t*, int, bool, hipStream_t);
I4_INST(I4_F16, I4_F32) I4_INST(I4_F16, I4_F16) I4_INST(I4_F16, I4_BF16)
I4_INST(I4_BF16, I4_F32) I4_INST(I4_BF16, I4_F16) I4_INST(I4_BF16, I4_BF16)
#undef I4_INST

}  // namespace i4
