// Fused int4 MoE block for gfx950 (replaces FusedPackedMoE.forward,
// src/duplex/streaming/fused_packed_moe.py:191-263), host pipeline and the
// small kernels around the expert projections.
//
// Decode (T = 1), three launches:
//   router logits (+ RMSNorm) -> gate_up<route> -> down + combine
// on CT rows (i4_moe_ct.hip) or on tiles (i4_moe_decode.hip), whichever
// layout the block's primary weights are in.  Decode is latency-bound and
// reads best as whole CT rows in narrow workgroups; the MFMA kernels need
// tiles, so a block may carry both (a tile copy costs one more copy of the
// weights, which HBM holds easily).
//
// Prefill / chunks (T > 1):
//   [RMSNorm] -> router logits -> top-k -> k_group -> MFMA gate_up (small and
//   large entries) -> MFMA down (small and large) -> k_moe_combine
// k_group sorts the T*topk (token, slot) pairs by expert (stable in token
// order): experts with <= 16 tokens become one small entry, larger ones
// entries of <= 64 tokens, so each weight tile is streamed once per entry
// instead of once per token (the reference loops over tokens,
// fused_packed_moe.py:231).  With T <= 64 every expert is cut into small
// entries and the large-entry launches are skipped.  The MFMA kernels are in
// i4_moe_mfma.hip.
#include "i4_common.h"
#include "i4_launch.h"
#include "i4_moe_launch.h"
#include "i4_topk.h"

namespace i4 {

static constexpr int WG = 256;
static constexpr int TCHUNK = 1024;  // tokens handled by one pass of the pipeline

// out[t] = residual[t] + sum_j w[t][j] ys[t][j] in slot order, ys [T * topk][H]
// in the activation dtype (each expert's output rounded as the reference rounds
// it, fused_packed_moe.py:262; half the bytes of fp32 through HBM), the sum in
// fp32.  KMAX >= topk slots are loaded unconditionally (indices clamped) so that
// all loads of a thread are in flight together.
template <int XT, int KMAX>
__global__ __launch_bounds__(WG) void k_moe_combine(const uint16_t* __restrict__ ys,
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
    yv[j] = Half<XT>::to_f32(ys[(int64_t)s * H + n]);
  }
  float y = 0.f;
#pragma unroll
  for (int j = 0; j < KMAX; ++j)
    if (j < topk) y += wv[j] * ((unsigned)sl[j] < (unsigned)E ? yv[j] : __builtin_nanf(""));
  const float r = residual ? Half<XT>::to_f32(rraw) : 0.f;
  if ((int64_t)blockIdx.x * WG + threadIdx.x < (int64_t)T * H) out[i] = Half<XT>::from_f32(r + y);
}


// ---------------------------------------------------------------------------
// Sort (token, slot) pairs by expert, stable in token order, and cut them
// into two lists: experts with <= lo_max tokens get entries of <= lo_chunk
// tokens in `entries`, the others entries of <= MF_TOK tokens in
// `mf_entries`.  One workgroup of 1024 threads (E <= 1024):
//   bits[w][e]: bit b set <=> token 32w + b selected expert e
//   pre [w][e]: popcount of bits[0..w)[e]
// (word-major, so the thread of expert e and its neighbours read adjacent words)
// and thread e owns expert e for the three exclusive prefix sums (tokens,
// first-list entries, second-list entries), done as wave scans plus a sum of
// the totals of the waves before its own.
//
// Inclusive prefix sum over the 64 lanes of a wave in DPP: shifts by 1, 2, 4
// and 8 lanes within each row of 16 (a lane with no source adds 0), then lane
// 15's total broadcast to rows 1 and 3 and lane 31's to rows 2 and 3 (the GCN
// wave scan of AMD's cross-lane operations guide).
__device__ inline int wave_incl_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true);   // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true);   // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);   // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true);   // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return v;
}

// One pass over a thread's (token, slot) pairs, SPT of them loaded before any
// is used (a loop that loads and uses one pair per turn waits a whole memory
// round trip per pair).  f(s, e) runs for every pair s < ns with its expert e.
template <int SPT, class F>
__device__ inline void for_pairs(const int32_t* sel, int ns, F f) {
  const int tid = threadIdx.x, nt = blockDim.x;
  for (int s0 = 0; s0 < ns; s0 += SPT * nt) {
    int ev[SPT];
#pragma unroll
    for (int u = 0; u < SPT; ++u) ev[u] = sel[min(s0 + u * nt + tid, ns - 1)];
#pragma unroll
    for (int u = 0; u < SPT; ++u) {
      const int s = s0 + u * nt + tid;
      if (s < ns) f(s, ev[u]);
    }
  }
}
template <class F> __device__ inline void pairs(const int32_t* sel, int ns, F f) {
  const int nt = blockDim.x;
  if (ns <= nt) for_pairs<1>(sel, ns, f);
  else if (ns <= 4 * nt) for_pairs<4>(sel, ns, f);
  else for_pairs<8>(sel, ns, f);
}

__device__ inline void group_body(const int32_t* sel, int T, int topk, int E, int lo_max,
                                  int lo_chunk, int32_t* __restrict__ perm,
                                  int4* __restrict__ entries, int* __restrict__ n_entries,
                                  int4* __restrict__ mf_entries, int* __restrict__ n_mf_entries,
                                  unsigned char* lds) {
  __shared__ int s_wsum[3][16];
  const int TW = (T + 31) >> 5;
  u32* bits = (u32*)lds;
  u32* pre = bits + E * TW;
  const int tid = threadIdx.x, nt = blockDim.x, wave = tid >> 6, lane = tid & 63;
  const int ns = T * topk;
  // capacities of the lists (the workspace holds E + T topk and E + T topk / MF_TOK + 1);
  // every index is checked against them, so no store can leave its buffer
  const int cap_s = E + ns, cap_m = E + ns / MF_TOK + 1;
  for (int i = tid; i < E * TW; i += nt) bits[i] = 0u;
  __syncthreads();
  pairs(sel, ns, [&](int s, int e) {
    const int t = s / topk;
    if ((unsigned)e < (unsigned)E) atomicOr(&bits[(t >> 5) * E + e], 1u << (t & 31));
  });
  __syncthreads();
  int c = 0;
  if (tid < E) {
    for (int w0 = 0; w0 < TW; w0 += 4) {  // four words read before any is counted
      u32 b[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) b[u] = bits[min(w0 + u, TW - 1) * E + tid];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (w0 + u < TW) {
          pre[(w0 + u) * E + tid] = (u32)c;
          c += __popc(b[u]);
        }
      }
    }
  }
  const bool big = c > lo_max;
  const int ne = big ? 0 : (c + lo_chunk - 1) / lo_chunk;
  const int nm = big ? (c + MF_TOK - 1) / MF_TOK : 0;
  const int ic = wave_incl_scan(c), ie = wave_incl_scan(ne), im = wave_incl_scan(nm);
  if (lane == 63) {
    s_wsum[0][wave] = ic;
    s_wsum[1][wave] = ie;
    s_wsum[2][wave] = im;
  }
  __syncthreads();
  // totals of the waves before this one: lane v < wave reads wave v's, then a sum
  const int nw = nt >> 6;
  const bool before = lane < wave && lane < nw;
  const int wl = min(lane, 15);
  const int bc = (int)group_sum<64>((float)(before ? s_wsum[0][wl] : 0));
  const int be = (int)group_sum<64>((float)(before ? s_wsum[1][wl] : 0));
  const int bm = (int)group_sum<64>((float)(before ? s_wsum[2][wl] : 0));
  const int off = bc + ic - c, eoff = be + ie - ne, moff = bm + im - nm;
  if (tid == nt - 1) {  // the last thread's inclusive sums are the totals
    *n_entries = min(be + ie, cap_s);
    *n_mf_entries = min(bm + im, cap_m);
  }
  int* s_off = (int*)(pre + E * TW);  // [E]
  if (tid < E) s_off[tid] = off;
  __syncthreads();
  pairs(sel, ns, [&](int s, int e) {
    const int t = s / topk;
    if ((unsigned)e < (unsigned)E) {
      const u32 word = bits[(t >> 5) * E + e];
      const int below = __popc(word & ((1u << (t & 31)) - 1u));
      const int at = s_off[e] + (int)pre[(t >> 5) * E + e] + below;
      if ((unsigned)at < (unsigned)ns) perm[at] = s;
    }
  });
  if (tid < E) {
    if (big) {
      for (int q = 0; q < nm; ++q)
        if (moff + q < cap_m)
          mf_entries[moff + q] = int4{tid, off + q * MF_TOK, min(MF_TOK, c - q * MF_TOK), 0};
    } else {
      for (int q = 0; q < ne; ++q)
        if (eoff + q < cap_s)
          entries[eoff + q] = int4{tid, off + q * lo_chunk, min(lo_chunk, c - q * lo_chunk), 0};
    }
  }
}

__global__ __launch_bounds__(1024) void k_group(const int32_t* __restrict__ sel, int T, int topk,
                                                int E, int lo_max, int lo_chunk,
                                                int32_t* __restrict__ perm,
                                                int4* __restrict__ entries,
                                                int* __restrict__ n_entries,
                                                int4* __restrict__ mf_entries,
                                                int* __restrict__ n_mf_entries,
                                                int32_t* __restrict__ status,
                                                u32* __restrict__ epoch) {
  extern __shared__ __align__(16) unsigned char lds[];
  if (status && threadIdx.x == 0) *status = I4_OK;  // nothing before this launch waits
  // the routing words of the next call carry another tag (k_router_topk_t)
  if (epoch && threadIdx.x == 0) *epoch = *epoch + 1u;
  group_body(sel, T, topk, E, lo_max, lo_chunk, perm, entries, n_entries, mf_entries,
             n_mf_entries, lds);
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
  int4* entries;  // small MFMA entries (<= MF_SMALL tokens)
  int* n_entries;
  int4* mf_entries;  // large MFMA entries (<= MF_TOK tokens)
  int* n_mf_entries;
  int32_t* status;  // I4_OK or I4_ERR_HANDOFF (i4_moe_status_offset)
  u32* epoch;
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
  // the tag epoch of the fused routing's words first, at the same offset for every T, so
  // that no other layout of the workspace writes over it
  m.epoch = (u32*)take(4);
  // [Tc][E] half logits, or [Tc][E / 2] (value pair, tag) words of the fused routing
  m.logits = take((size_t)Tc * E * 4);
  m.xn = (uint16_t*)take((size_t)Tc * H * 2);
  m.sel = (int32_t*)take(Tk * 4);
  m.w = (float*)take(Tk * 4);
  m.act = (uint16_t*)take(Tk * I * 2);
  m.ys = Tc > 1 ? (float*)take(Tk * H * 2) : nullptr;  // [Tk][H] in the activation dtype
  m.perm = (int32_t*)take(Tk * 4);
  m.entries = (int4*)take((E + Tk) * sizeof(int4));
  m.n_entries = (int*)take(4);
  m.mf_entries = (int4*)take((E + Tk / MF_TOK + 1) * sizeof(int4));
  m.n_mf_entries = (int*)take(4);
  m.status = (int32_t*)take(4);
  m.bytes = o;
  return m;
}

TW to_tw(const i4_qweight& w) {
  TW q;
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

struct MoeOps {
  int (*gate_up)(const GateUpArgs&, const TW&, int, hipStream_t);
  int (*down_m1)(const void*, int, const int32_t*, const float*, const TW&, const void*, void*,
                 hipStream_t);
  int (*gate_up_ct)(const GateUpArgs&, const TW&, int, hipStream_t);
  int (*down_m1_ct)(const void*, int, const int32_t*, const float*, const TW&, const void*, void*,
                    hipStream_t);
  int (*mfma_gate_up)(bool, int, const void*, int, int, const int4*, const int*, const int32_t*,
                      const TW&, int, void*, hipStream_t);
  int (*mfma_down)(bool, int, const void*, int, const int4*, const int*, const int32_t*,
                   const TW&, void*, hipStream_t);
  int (*moe_m1_ct)(const GateUpArgs&, const TW*, const TW&, const void*, void*, int32_t*, int,
                   hipStream_t);
  int (*mfma_mixed)(bool, int, int, const void*, int, int, const int4*, const int*, const int4*,
                    const int*, const int32_t*, const TW&, int, void*, hipStream_t);
  int (*moe_m1x_ct)(const GateUpArgs&, const TW&, const TW&, void*, int32_t*, int, bool,
                    hipStream_t);
  int (*mfma_gd)(int, const void*, int, int, const int4*, const int*, const int32_t*, const TW&,
                 const TW&, int, void*, void*, int32_t*, int, bool, hipStream_t);
};

template <int XT, int ST> constexpr MoeOps moe_ops() {
  return MoeOps{&launch_gate_up<XT, ST>,     &launch_down_m1<XT, ST>,
                &launch_gate_up_ct<XT, ST>,  &launch_down_m1_ct<XT, ST>,
                &launch_mfma_gate_up<XT, ST>, &launch_mfma_down<XT, ST>,
                &launch_moe_m1_ct<XT, ST>,   &launch_mfma_mixed<XT, ST>,
                &launch_moe_m1x_ct<XT, ST>,  &launch_mfma_gd<XT, ST>};
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

// a weight the decode kernels can read: CT rows or tiles, K <= 4096
int check_decode(const i4_qweight* in, i4_qweight* w) {
  int rc = i4_check_weight(in, w);
  if (rc) return rc;
  if (w->layout != I4_LAYOUT_CT && w->layout != I4_LAYOUT_TILE) return I4_ERR_LAYOUT;
  if (w->K > 4096) return I4_ERR_SHAPE;
  return I4_OK;
}

bool present(const i4_qweight& w) { return w.packed != nullptr; }

// Validate a block.  gu / dn: the decode weights; tgu / tdn: the tile
// weights of the MFMA path (the tile copies, or gu / dn when those are tiles;
// layout -1 when the block has none).
int check_moe(const i4_moe_weights* mw, int x_dtype, int T, int topk, i4_qweight* gu,
              i4_qweight* dn, i4_qweight* tgu, i4_qweight* tdn) {
  if (!mw) return I4_ERR_NULL;
  int rc = check_decode(&mw->gate_up, gu);
  if (rc) return rc;
  rc = check_decode(&mw->down, dn);
  if (rc) return rc;
  if (gu->layout != dn->layout) return I4_ERR_LAYOUT;
  if (x_dtype != I4_F16 && x_dtype != I4_BF16) return I4_ERR_DTYPE;
  const int H = gu->K, I = dn->K, E = gu->E;
  if (gu->N != 2 * I || dn->N != H || dn->E != E) return I4_ERR_SHAPE;
  if (T < 1 || E > 512 || topk < 1 || topk > E || topk > 16) return I4_ERR_SHAPE;
  if (present(mw->gate_up_tile) != present(mw->down_tile)) return I4_ERR_NULL;
  if (present(mw->gate_up_tile)) {
    rc = check_decode(&mw->gate_up_tile, tgu);
    if (rc) return rc;
    rc = check_decode(&mw->down_tile, tdn);
    if (rc) return rc;
    if (tgu->layout != I4_LAYOUT_TILE || tdn->layout != I4_LAYOUT_TILE) return I4_ERR_LAYOUT;
    if (tgu->E != E || tgu->N != gu->N || tgu->K != H || tdn->E != E || tdn->N != H ||
        tdn->K != I)
      return I4_ERR_SHAPE;
  } else if (gu->layout == I4_LAYOUT_TILE) {
    *tgu = *gu;
    *tdn = *dn;
  } else {
    tgu->layout = tdn->layout = -1;
  }
  if (T > 1 && tgu->layout != I4_LAYOUT_TILE) return I4_ERR_LAYOUT;  // MFMA kernels read tiles
  if (tgu->layout == I4_LAYOUT_TILE) {
    // column tiles of the MFMA kernels: 32 * MF_NB row pairs / 64 * MF_NB rows
    if (I % (32 * MF_NB) != 0 || H % (64 * MF_NB) != 0) return I4_ERR_SHAPE;
    if (tgu->scale_dtype != gu->scale_dtype || tdn->scale_dtype != dn->scale_dtype)
      return I4_ERR_DTYPE;
  }
  if (gu->layout == I4_LAYOUT_TILE && (I % 16 != 0 || H % 16 != 0)) return I4_ERR_SHAPE;
  return I4_OK;
}

// reset: this chunk's first kernel clears the status word (the first chunk of
// a call, the first layer of a stack), so a later give-up is not overwritten
// max_polls / mode (i4_moe_forward_bounded): the bound of the T <= 64 waits; mode 1: the
// grouped launch's down workgroups alone, 2: the routing launch's ranking waves alone
int moe_chunk(const void* x, int xt, int T, const i4_moe_weights* mw, const i4_qweight& gu,
              const i4_qweight& dn, const i4_qweight& tg, const i4_qweight& td, int topk,
              int renorm, const void* logits, const void* residual, void* out, int32_t* sel_out,
              float* w_out, const MoeWs& ws, bool reset, hipStream_t s,
              int max_polls = kHandoffPolls, int mode = 0) {
  const bool down_only = mode == 1, rank_only = mode == 2;
  int32_t* st_reset = reset && !rank_only ? ws.status : nullptr;
  const int H = gu.K, I = dn.K, E = gu.E;
  MoeOps ops;
  if (!pick_ops(xt, gu.scale_dtype, dn.scale_dtype, &ops)) return I4_ERR_DTYPE;
  int rc;
  int32_t* sel = sel_out ? sel_out : ws.sel;
  float* wts = w_out ? w_out : ws.w;
  const bool ct = gu.layout == I4_LAYOUT_CT;
  if (T == 1) {
    // decode: router -> gate_up (ranks the logits itself) -> down + combine;
    // on CT rows with the router in the block, both expert projections run
    // as one launch whose down workgroups wait for act in the kernel (the
    // router launch marks act pending first)
    const bool one = ct && mw->router_w && moe_m1_ct_fits(topk, H, I);
    const void* lg = logits;
    if (mw->router_w) {
      rc = i4_launch_router_logits(x, xt, 1, H, mw->router_w, E, mw->norm_w, mw->norm_eps,
                                   mw->norm_w ? ws.xn : nullptr, ws.logits, s,
                                   one ? ws.act : nullptr, one ? topk * I / 8 : 0, st_reset);
      if (rc) return rc;
      lg = ws.logits;
      if (mw->norm_w) x = ws.xn;  // the experts run on RMSNorm(x); residual is untouched
      st_reset = nullptr;
    }
    const GateUpArgs a{true, topk, topk, E, renorm, x, sel, lg, wts, ws.act, st_reset};
    if (one) {
      const TW tg_ = to_tw(gu);
      return ops.moe_m1_ct(a, &tg_, to_tw(dn), residual, out, ws.status, kHandoffPolls, s);
    }
    rc = (ct ? ops.gate_up_ct : ops.gate_up)(a, to_tw(gu), I, s);
    if (rc) return rc;
    return (ct ? ops.down_m1_ct : ops.down_m1)(ws.act, topk, sel, wts, to_tw(dn), residual, out, s);
  }
  const TW tgu = to_tw(tg), tdn = to_tw(td);
  const int Tk = T * topk;
  const bool one_list = T <= ONE_LIST_T;
  // T <= 64 with one group size for both projections: gate_up and down share a launch
  // whose down workgroups take act over inside it; the routing launch sets act pending.
  // (The same for both entry lists above 64 tokens measured no faster at M = 512: setting
  // 6.3 MB pending and writing the activations through cost what the launch saved.)
  const bool gd = one_list && tgu.gshift == tdn.gshift;
  void* pend = gd ? ws.act : nullptr;
  const int n_pend = gd ? (int)((int64_t)Tk * I / 8) : 0;
  // 2..64 tokens with the router in the block: router and top-k as one launch whose
  // ranking waves take the logits over inside it (k_router_topk_t)
  const bool fused = mw->router_w && T >= 2 && T <= 64 && E <= 128 && E % 4 == 0;
  const void* lg = logits;
  if (fused) {
    rc = i4_launch_router_topk(x, xt, T, H, mw->router_w, E, mw->norm_w, mw->norm_eps,
                               mw->norm_w ? ws.xn : nullptr, (u32*)ws.logits, ws.epoch, topk,
                               renorm, sel, wts, pend, n_pend, st_reset, ws.status,
                               rank_only ? max_polls : kHandoffPolls, rank_only, s);
    if (rc) return rc;
    if (mw->norm_w) x = ws.xn;
    st_reset = nullptr;
  } else if (mw->router_w) {
    rc = i4_launch_router_logits(x, xt, T, H, mw->router_w, E, mw->norm_w, mw->norm_eps,
                                 mw->norm_w ? ws.xn : nullptr, ws.logits, s);
    if (rc) return rc;
    lg = ws.logits;
    if (mw->norm_w) x = ws.xn;
  }
  const int TW_ = (T + 31) / 32;
  const size_t glds = (size_t)2 * E * TW_ * 4 + (size_t)E * 4;
  // T <= MF_TOK: no expert has more tokens than one large entry holds, and
  // small entries of <= MF_SMALL tokens cover every expert in one launch per
  // projection; above, experts with > MF_SMALL tokens take large entries.
  // Otherwise top-k on T / 4 workgroups (one token per wave), then the grouping: ranking
  // every token inside the one grouping workgroup queued the waves' scalar bisection steps
  // on one CU's scalar unit (5 us of the launch at T = 32; separate launches 1.5 us faster)
  if (!fused) {
    rc = i4_launch_topk(lg, xt, T, E, topk, renorm, sel, wts, nullptr, 0, s, pend, n_pend);
    if (rc) return rc;
  }
  hipLaunchKernelGGL(k_group, dim3(1), dim3(1024), glds, s, sel, T, topk, E,
                     one_list ? T : MF_SMALL, MF_SMALL, ws.perm, ws.entries, ws.n_entries,
                     ws.mf_entries, ws.n_mf_entries, st_reset, fused ? ws.epoch : nullptr);
  if (hipGetLastError() != hipSuccess) return I4_ERR_LAUNCH;
  // entry counts: sum over experts of ceil(n_e / 16) <= min(E, Tk) + Tk / 16
  const int max_s = (E < Tk ? E : Tk) + (one_list ? Tk / MF_SMALL : 0);
  const int max_b = (E < Tk / (MF_SMALL + 1) ? E : Tk / (MF_SMALL + 1)) + Tk / MF_TOK + 1;
  if (gd) {
    rc = ops.mfma_gd(max_s, x, T, topk, ws.entries, ws.n_entries, ws.perm, tgu, tdn, I, ws.act,
                     ws.ys, ws.status, rank_only ? kHandoffPolls : max_polls, down_only, s);
    if (rc) return rc;
  } else if (one_list) {
    rc = ops.mfma_gate_up(true, max_s, x, T, topk, ws.entries, ws.n_entries, ws.perm, tgu, I,
                          ws.act, s);
    if (rc) return rc;
    rc = ops.mfma_down(true, max_s, ws.act, Tk, ws.entries, ws.n_entries, ws.perm, tdn, ws.ys, s);
    if (rc) return rc;
  } else {  // large and small entries of a projection share one launch
    rc = ops.mfma_mixed(true, max_b, max_s, x, T, topk, ws.mf_entries, ws.n_mf_entries,
                        ws.entries, ws.n_entries, ws.perm, tgu, I, ws.act, s);
    if (rc) return rc;
    rc = ops.mfma_mixed(false, max_b, max_s, ws.act, Tk, topk, ws.mf_entries, ws.n_mf_entries,
                        ws.entries, ws.n_entries, ws.perm, tdn, I, ws.ys, s);
    if (rc) return rc;
  }
  const int64_t tot = (int64_t)T * H;
  dim3 cg((unsigned)((tot + WG - 1) / WG));
#define I4_COMB_CASE(XT_, KM_)                                                                 \
  hipLaunchKernelGGL((k_moe_combine<XT_, KM_>), cg, dim3(WG), 0, s, (const uint16_t*)ws.ys, wts, \
                     sel, T, topk, E, H, (const uint16_t*)residual, (uint16_t*)out)
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

// i4_moe_forward with the status reset under the caller's control (the stack
// clears it in its first layer only, so a give-up in any layer stays visible)
int moe_forward_impl(const void* x, int x_dtype, int T, const i4_moe_weights* weights, int topk,
                     int renorm, const void* logits, const void* residual, void* out,
                     int32_t* sel_out, float* w_out, void* workspace, size_t workspace_bytes,
                     bool reset, hipStream_t stream, int32_t* status = nullptr,
                     int max_polls = kHandoffPolls, int mode = 0) {
  i4_qweight gu, dn, tg, td;
  int rc = check_moe(weights, x_dtype, T, topk, &gu, &dn, &tg, &td);
  if (rc) return rc;
  if (!x || !out) return I4_ERR_NULL;
  if (!weights->router_w && !logits) return I4_ERR_NULL;
  if (weights->norm_w && !weights->router_w) return I4_ERR_NULL;
  if ((uintptr_t)weights->norm_w & 15) return I4_ERR_ALIGN;
  if (((uintptr_t)x & 15) || ((uintptr_t)out & 15) || ((uintptr_t)residual & 15))
    return I4_ERR_ALIGN;
  const int H = gu.K, I = dn.K, E = gu.E;
  const MoeWs need = carve(nullptr, T, H, I, E, topk);
  if (!workspace || workspace_bytes < need.bytes) return I4_ERR_WORKSPACE;
  if ((uintptr_t)workspace & 255) return I4_ERR_ALIGN;
  MoeWs ws = carve(workspace, T, H, I, E, topk);
  if (status) ws.status = status;  // the caller's status word instead of the workspace's
  for (int t0 = 0; t0 < T; t0 += TCHUNK) {
    const int Tc = T - t0 < TCHUNK ? T - t0 : TCHUNK;
    const char* xs = (const char*)x + (size_t)t0 * H * 2;
    const void* lg = logits ? (const char*)logits + (size_t)t0 * E * 2 : nullptr;
    const void* rs = residual ? (const char*)residual + (size_t)t0 * H * 2 : nullptr;
    void* os = (char*)out + (size_t)t0 * H * 2;
    rc = moe_chunk(xs, x_dtype, Tc, weights, gu, dn, tg, td, topk, renorm, lg, rs, os,
                   sel_out ? sel_out + (size_t)t0 * topk : nullptr,
                   w_out ? w_out + (size_t)t0 * topk : nullptr, ws, reset && t0 == 0, stream,
                   max_polls, mode);
    if (rc) return rc;
  }
  return I4_OK;
}

}  // namespace

namespace i4 {

int moe_decode_bufs(const i4_moe_weights* mw, int x_dtype, int topk, void* ws, size_t ws_bytes,
                    MoeDecodeBufs* b) {
  i4_qweight gu, dn, tg, td;
  int rc = check_moe(mw, x_dtype, 1, topk, &gu, &dn, &tg, &td);
  if (rc) return rc;
  if (!mw->router_w || !mw->norm_w) return I4_ERR_NULL;
  if (gu.layout != I4_LAYOUT_CT) return I4_ERR_LAYOUT;
  const int H = gu.K, I = dn.K, E = gu.E;
  if ((H != 1024 && H != 2048) || !moe_m1_ct_fits(topk, H, I)) return I4_ERR_SHAPE;
  if (((uintptr_t)mw->router_w & 15) || ((uintptr_t)mw->norm_w & 15)) return I4_ERR_ALIGN;
  if (!ws || ws_bytes < carve(nullptr, 1, H, I, E, topk).bytes) return I4_ERR_WORKSPACE;
  if ((uintptr_t)ws & 255) return I4_ERR_ALIGN;
  MoeOps ops;
  if (!pick_ops(x_dtype, gu.scale_dtype, dn.scale_dtype, &ops)) return I4_ERR_DTYPE;
  const MoeWs w = carve(ws, 1, H, I, E, topk);
  b->logits = (uint16_t*)w.logits;
  b->xn = w.xn;
  b->act = (u32x4*)w.act;
  b->n_act = topk * I / 8;
  b->status = w.status;
  b->w = w.w;
  b->H = H;
  b->I = I;
  b->E = E;
  b->gate_up = gu;
  b->down = dn;
  return I4_OK;
}

int moe_decode_experts(const MoeDecodeBufs& b, int x_dtype, int topk, int renorm,
                       const void* residual, void* out, void* ws, hipStream_t s) {
  const i4_qweight& gu = b.gate_up;
  const i4_qweight& dn = b.down;
  const MoeWs w = carve(ws, 1, gu.K, dn.K, gu.E, topk);
  MoeOps ops;
  if (!pick_ops(x_dtype, gu.scale_dtype, dn.scale_dtype, &ops)) return I4_ERR_DTYPE;
  // the status word was reset before the router launch, which may have reported in it
  const GateUpArgs a{true, topk, topk, gu.E, renorm, w.xn, w.sel, w.logits, w.w, w.act, nullptr};
  const TW tg = to_tw(gu);
  return ops.moe_m1_ct(a, &tg, to_tw(dn), residual, out, w.status, kHandoffPolls, s);
}

int moe_decode_experts_x(const MoeDecodeBufs& b, int x_dtype, int topk, int renorm, void* ypart,
                         void* ws, hipStream_t s) {
  const i4_qweight& gu = b.gate_up;
  const i4_qweight& dn = b.down;
  if (!moe_m1x_ct_fits(topk, gu.K, dn.K)) return I4_ERR_SHAPE;
  const MoeWs w = carve(ws, 1, gu.K, dn.K, gu.E, topk);
  MoeOps ops;
  if (!pick_ops(x_dtype, gu.scale_dtype, dn.scale_dtype, &ops)) return I4_ERR_DTYPE;
  const GateUpArgs a{true, topk, topk, gu.E, renorm, w.xn, w.sel, w.logits, w.w, w.act, nullptr};
  return ops.moe_m1x_ct(a, to_tw(gu), to_tw(dn), ypart, w.status, kHandoffPolls, false, s);
}

int moe_forward_status(const void* x, int x_dtype, int T, const i4_moe_weights* weights,
                       int topk, int renorm, const void* logits, const void* residual, void* out,
                       int32_t* sel_out, float* w_out, void* workspace, size_t workspace_bytes,
                       int32_t* status, hipStream_t stream) {
  if ((uintptr_t)status & 3) return I4_ERR_ALIGN;
  return moe_forward_impl(x, x_dtype, T, weights, topk, renorm, logits, residual, out, sel_out,
                          w_out, workspace, workspace_bytes, true, stream, status);
}

}  // namespace i4

namespace {

// stack workspace beyond the T = 1 MoE workspace: the hidden state between layers;
// at T = 1 a second one and the slot outputs [topk][H] of the XCD-local path
size_t stack_extra_bytes(int T, int H, int topk) {
  const size_t h = al256((size_t)T * H * 2);
  return T == 1 ? 2 * h + al256((size_t)topk * H * 2) : h;
}

// every layer of a T = 1 stack can run the XCD-local experts launch (validated blocks)
bool stack_xcd_local(const i4_moe_weights* layers, int n, int xt, int topk) {
  for (int l = 0; l < n; ++l) {
    const i4_moe_weights& w = layers[l];
    const int H = w.gate_up.K, I = w.down.K;
    MoeOps ops;
    if (w.gate_up.layout != I4_LAYOUT_CT || !w.router_w || (H != 1024 && H != 2048) ||
        !moe_m1x_ct_fits(topk, H, I) || !pick_ops(xt, w.gate_up.scale_dtype,
                                                  w.down.scale_dtype, &ops))
      return false;
  }
  return true;
}

// One validated block of the XCD-local decode path.
struct XBlock {
  i4_qweight gu, dn;
  MoeOps ops;
  int H, I, E;
};
int xblock(const i4_moe_weights* mw, int xt, int topk, XBlock* b) {
  i4_qweight tg, td;
  int rc = check_moe(mw, xt, 1, topk, &b->gu, &b->dn, &tg, &td);
  if (rc) return rc;
  if (!mw->router_w) return I4_ERR_NULL;
  if (b->gu.layout != I4_LAYOUT_CT) return I4_ERR_LAYOUT;
  b->H = b->gu.K;
  b->I = b->dn.K;
  b->E = b->gu.E;
  if ((b->H != 1024 && b->H != 2048) || !moe_m1x_ct_fits(topk, b->H, b->I)) return I4_ERR_SHAPE;
  if (((uintptr_t)mw->router_w & 15) || ((uintptr_t)mw->norm_w & 15)) return I4_ERR_ALIGN;
  if (!pick_ops(xt, b->gu.scale_dtype, b->dn.scale_dtype, &b->ops)) return I4_ERR_DTYPE;
  return I4_OK;
}

// the router launch of a layer: on res itself (ypart == nullptr, the first layer), or
// completing the previous layer first, h = res + sum_j w_j ypart[j] into h_out
int x_route(const void* res, int xt, const void* ypart, const i4_moe_weights* mw,
            const XBlock& b, int topk, void* h_out, const MoeWs& ws, bool reset, hipStream_t s) {
  uint16_t* xn = mw->norm_w ? ws.xn : nullptr;
  int32_t* st = reset ? ws.status : nullptr;
  if (!ypart)
    return i4_launch_router_logits(res, xt, 1, b.H, mw->router_w, b.E, mw->norm_w, mw->norm_eps,
                                   xn, ws.logits, s, ws.act, topk * b.I / 8, st);
  return i4_launch_router_sum(res, ypart, ws.w, topk, h_out, xt, b.H, mw->router_w, b.E,
                              mw->norm_w, mw->norm_eps, xn, ws.logits, s, ws.act,
                              topk * b.I / 8, st);
}

// the experts launch of a layer: h is the routed row (read when the block has no norm)
int x_experts(const void* h, const i4_moe_weights* mw, const XBlock& b, int topk, int renorm,
              void* ypart, const MoeWs& ws, int max_polls, bool down_only, hipStream_t s) {
  const void* x = mw->norm_w ? (const void*)ws.xn : h;
  const GateUpArgs a{true, topk, topk, b.E, renorm, x, ws.sel, ws.logits, ws.w, ws.act, nullptr};
  return b.ops.moe_m1x_ct(a, to_tw(b.gu), to_tw(b.dn), ypart, ws.status, max_polls, down_only, s);
}

// T = 1 stack on the XCD-local experts launch.  Layer l's router launch first
// completes layer l - 1 (h_l = h_{l-1} + sum_j w_j y_j, written to hb[l % 2]) and
// routes h_l; the experts launch leaves its slot outputs in ypart and its routing
// weights in ws.w; one more launch completes the last layer into out.  The router
// launch of layer 0 clears the status word, so a wait that gives up in any layer
// stays visible.
int stack_m1x(const void* x, int xt, const i4_moe_weights* layers, int n, int topk, int renorm,
              void* out, const MoeWs& ws, uint16_t* hb0, uint16_t* hb1, uint16_t* ypart,
              hipStream_t s) {
  const void* h = x;  // h_l, the input of layer l
  for (int l = 0; l < n; ++l) {
    XBlock b;
    int rc = xblock(&layers[l], xt, topk, &b);
    if (rc) return rc;
    uint16_t* hl = (l % 2) ? hb1 : hb0;
    rc = x_route(h, xt, l ? ypart : nullptr, &layers[l], b, topk, hl, ws, l == 0, s);
    if (rc) return rc;
    if (l) h = hl;
    rc = x_experts(h, &layers[l], b, topk, renorm, ypart, ws, kHandoffPolls, false, s);
    if (rc) return rc;
  }
  return i4_launch_moe_sum(h, ypart, ws.w, topk, xt, layers[0].gate_up.K, out, s);
}

}  // namespace

extern "C" {

size_t i4_moe_workspace_bytes(int T, int H, int I, int E, int topk) {
  if (T < 1 || H < 1 || I < 1 || E < 1 || topk < 1) return 0;
  return carve(nullptr, T, H, I, E, topk).bytes;
}

size_t i4_moe_status_offset(int T, int H, int I, int E, int topk) {
  if (T < 1 || H < 1 || I < 1 || E < 1 || topk < 1) return 0;
  char* const base = (char*)(uintptr_t)4096;  // carve() lays out from any aligned base
  return (size_t)((char*)carve(base, T, H, I, E, topk).status - base);
}

int i4_moe_forward(const void* x, int x_dtype, int T, const i4_moe_weights* weights, int topk,
                   int renorm, const void* logits, const void* residual, void* out,
                   int32_t* sel_out, float* w_out, void* workspace, size_t workspace_bytes,
                   hipStream_t stream) {
  return moe_forward_impl(x, x_dtype, T, weights, topk, renorm, logits, residual, out, sel_out,
                          w_out, workspace, workspace_bytes, true, stream);
}

int i4_moe_forward_bounded(const void* x, int x_dtype, int T, const i4_moe_weights* weights,
                           int topk, int renorm, const void* logits, const void* residual,
                           void* out, void* workspace, size_t workspace_bytes, int max_polls,
                           int down_only, hipStream_t stream) {
  if (!weights) return I4_ERR_NULL;
  // only the fused T <= 64 launch waits: 2..64 tokens, one group size for both projections
  if (T < 2 || T > ONE_LIST_T || max_polls < 0 || down_only < 0 || down_only > 2)
    return I4_ERR_SHAPE;
  const i4_qweight& g = weights->gate_up_tile.packed ? weights->gate_up_tile : weights->gate_up;
  const i4_qweight& d = weights->down_tile.packed ? weights->down_tile : weights->down;
  if (g.group != d.group) return I4_ERR_SHAPE;
  // mode 2 needs the fused routing launch: the router in the block, E <= 128, E % 4 == 0
  if (down_only == 2 && (!weights->router_w || logits || g.E > 128 || g.E % 4 != 0))
    return I4_ERR_SHAPE;
  return moe_forward_impl(x, x_dtype, T, weights, topk, renorm, logits, residual, out, nullptr,
                          nullptr, workspace, workspace_bytes, true, stream, nullptr, max_polls,
                          down_only);
}


int i4_moe_down_wait(const void* act, int x_dtype, const i4_qweight* down, const void* logits,
                     int E_r, int topk, int renorm, const void* residual, void* out,
                     int32_t* status, int max_polls, hipStream_t stream) {
  i4_qweight dn;
  int rc = check_decode(down, &dn);
  if (rc) return rc;
  if (!act || !logits || !out || !status) return I4_ERR_NULL;
  if (x_dtype != I4_F16 && x_dtype != I4_BF16) return I4_ERR_DTYPE;
  if (dn.layout != I4_LAYOUT_CT) return I4_ERR_LAYOUT;
  if (E_r < 1 || E_r > 512 || E_r > dn.E || topk < 1 || topk > E_r || max_polls < 0)
    return I4_ERR_SHAPE;
  if (!moe_m1_ct_fits(topk, dn.N, dn.K)) return I4_ERR_SHAPE;
  if (((uintptr_t)act & 15) || ((uintptr_t)out & 15) || ((uintptr_t)residual & 15) ||
      ((uintptr_t)status & 3))
    return I4_ERR_ALIGN;
  MoeOps ops;
  if (!pick_ops(x_dtype, dn.scale_dtype, dn.scale_dtype, &ops)) return I4_ERR_DTYPE;
  const GateUpArgs a{true, topk, topk, E_r, renorm, nullptr, nullptr, logits, nullptr,
                     const_cast<void*>(act), nullptr};
  return ops.moe_m1_ct(a, nullptr, to_tw(dn), residual, out, status, max_polls, stream);
}

int i4_moe_gate_up(const void* x, int x_dtype, const i4_qweight* gate_up, const int32_t* sel,
                   int topk, void* act, hipStream_t stream) {
  i4_qweight gu;
  int rc = check_decode(gate_up, &gu);
  if (rc) return rc;
  if (!x || !sel || !act) return I4_ERR_NULL;
  if (x_dtype != I4_F16 && x_dtype != I4_BF16) return I4_ERR_DTYPE;
  if (topk < 1 || topk > 65535 || gu.N % (gu.layout == I4_LAYOUT_TILE ? 32 : 2))
    return I4_ERR_SHAPE;
  if (((uintptr_t)x & 15) || ((uintptr_t)act & 15)) return I4_ERR_ALIGN;
  MoeOps ops;
  if (!pick_ops(x_dtype, gu.scale_dtype, gu.scale_dtype, &ops)) return I4_ERR_DTYPE;
  const GateUpArgs a{false, topk, topk, 0, 0, x, const_cast<int32_t*>(sel), nullptr, nullptr,
                     act, nullptr};
  return (gu.layout == I4_LAYOUT_CT ? ops.gate_up_ct : ops.gate_up)(a, to_tw(gu), gu.N / 2, stream);
}

int i4_moe_route_gate_up(const void* x, int x_dtype, const i4_qweight* gate_up,
                         const void* logits, int E_r, int topk, int renorm, int32_t* sel_out,
                         float* w_out, void* act, hipStream_t stream) {
  i4_qweight gu;
  int rc = check_decode(gate_up, &gu);
  if (rc) return rc;
  if (!x || !logits || !sel_out || !w_out || !act) return I4_ERR_NULL;
  if (x_dtype != I4_F16 && x_dtype != I4_BF16) return I4_ERR_DTYPE;
  if (E_r < 1 || E_r > 512 || E_r > gu.E || topk < 1 || topk > E_r || topk > 64 ||
      gu.N % (gu.layout == I4_LAYOUT_TILE ? 32 : 2))
    return I4_ERR_SHAPE;
  if (((uintptr_t)x & 15) || ((uintptr_t)act & 15)) return I4_ERR_ALIGN;
  MoeOps ops;
  if (!pick_ops(x_dtype, gu.scale_dtype, gu.scale_dtype, &ops)) return I4_ERR_DTYPE;
  const GateUpArgs a{true, topk, topk, E_r, renorm, x, sel_out, logits, w_out, act, nullptr};
  return (gu.layout == I4_LAYOUT_CT ? ops.gate_up_ct : ops.gate_up)(a, to_tw(gu), gu.N / 2, stream);
}

int i4_moe_down_combine(const void* act, int x_dtype, const i4_qweight* down, const int32_t* sel,
                        const float* w, int topk, const void* residual, void* out,
                        hipStream_t stream) {
  i4_qweight dn;
  int rc = check_decode(down, &dn);
  if (rc) return rc;
  if (!act || !sel || !w || !out) return I4_ERR_NULL;
  if (x_dtype != I4_F16 && x_dtype != I4_BF16) return I4_ERR_DTYPE;
  if (topk < 1 || topk > 16) return I4_ERR_SHAPE;
  if (((uintptr_t)act & 15) || ((uintptr_t)out & 15) || ((uintptr_t)residual & 15))
    return I4_ERR_ALIGN;
  MoeOps ops;
  if (!pick_ops(x_dtype, dn.scale_dtype, dn.scale_dtype, &ops)) return I4_ERR_DTYPE;
  return (dn.layout == I4_LAYOUT_CT ? ops.down_m1_ct : ops.down_m1)(act, topk, sel, w, to_tw(dn),
                                                                   residual, out, stream);
}

size_t i4_moe_stack_workspace_bytes(int T, int H, int I, int E, int topk) {
  const size_t m = i4_moe_workspace_bytes(T, H, I, E, topk);
  if (!m) return 0;
  return m + stack_extra_bytes(T, H, topk);
}

int i4_moe_stack_forward(const void* x, int x_dtype, int T, const i4_moe_weights* layers,
                         int n_layers, int topk, int renorm, void* out, void* workspace,
                         size_t workspace_bytes, hipStream_t stream) {
  if (!layers || !x || !out) return I4_ERR_NULL;
  if (n_layers < 1) return I4_ERR_SHAPE;
  i4_qweight gu, dn, tg, td;
  for (int l = 0; l < n_layers; ++l) {
    int rc = check_moe(&layers[l], x_dtype, T, topk, &gu, &dn, &tg, &td);
    if (rc) return rc;
    if (!layers[l].router_w) return I4_ERR_NULL;
  }
  int rc = check_moe(&layers[0], x_dtype, T, topk, &gu, &dn, &tg, &td);
  const int H = gu.K, I = dn.K, E = gu.E;
  for (int l = 1; l < n_layers; ++l)
    if (layers[l].gate_up.K != H || layers[l].down.K != I || layers[l].gate_up.E != E)
      return I4_ERR_SHAPE;
  const size_t mbytes = i4_moe_workspace_bytes(T, H, I, E, topk);
  if (!workspace || workspace_bytes < mbytes + stack_extra_bytes(T, H, topk))
    return I4_ERR_WORKSPACE;
  if ((uintptr_t)workspace & 255) return I4_ERR_ALIGN;
  void* buf = (char*)workspace + mbytes;
  if (T == 1 && stack_xcd_local(layers, n_layers, x_dtype, topk))
    return stack_m1x(x, x_dtype, layers, n_layers, topk, renorm, out,
                     carve(workspace, 1, H, I, E, topk), (uint16_t*)buf,
                     (uint16_t*)((char*)buf + al256((size_t)H * 2)),
                     (uint16_t*)((char*)buf + 2 * al256((size_t)H * 2)), stream);
  const void* h = x;
  for (int l = 0; l < n_layers; ++l) {
    void* dst = ((n_layers - 1 - l) % 2 == 0) ? out : buf;
    rc = moe_forward_impl(h, x_dtype, T, &layers[l], topk, renorm, nullptr, h, dst, nullptr,
                          nullptr, workspace, mbytes, l == 0, stream);
    if (rc) return rc;
    h = dst;
  }
  return I4_OK;
}


int i4_moe_route_sum(const void* res, int x_dtype, const void* ypart,
                     const i4_moe_weights* weights, int topk, void* h_out, int reset_status,
                     void* workspace, size_t workspace_bytes, hipStream_t stream) {
  XBlock b;
  int rc = xblock(weights, x_dtype, topk, &b);
  if (rc) return rc;
  if (!res || (ypart && !h_out)) return I4_ERR_NULL;
  if (((uintptr_t)res & 15) || ((uintptr_t)ypart & 15) || ((uintptr_t)h_out & 15))
    return I4_ERR_ALIGN;
  if (!workspace || workspace_bytes < carve(nullptr, 1, b.H, b.I, b.E, topk).bytes)
    return I4_ERR_WORKSPACE;
  if ((uintptr_t)workspace & 255) return I4_ERR_ALIGN;
  const MoeWs ws = carve(workspace, 1, b.H, b.I, b.E, topk);
  return x_route(res, x_dtype, ypart, weights, b, topk, h_out, ws, reset_status != 0, stream);
}

int i4_moe_experts_x(const void* h, int x_dtype, const i4_moe_weights* weights, int topk,
                     int renorm, void* ypart, int max_polls, int down_only, void* workspace,
                     size_t workspace_bytes, hipStream_t stream) {
  XBlock b;
  int rc = xblock(weights, x_dtype, topk, &b);
  if (rc) return rc;
  if (!ypart || (!weights->norm_w && !h)) return I4_ERR_NULL;
  if (((uintptr_t)ypart & 15) || ((uintptr_t)h & 15)) return I4_ERR_ALIGN;
  if (max_polls < 0) return I4_ERR_SHAPE;
  if (!workspace || workspace_bytes < carve(nullptr, 1, b.H, b.I, b.E, topk).bytes)
    return I4_ERR_WORKSPACE;
  if ((uintptr_t)workspace & 255) return I4_ERR_ALIGN;
  const MoeWs ws = carve(workspace, 1, b.H, b.I, b.E, topk);
  return x_experts(h, weights, b, topk, renorm, ypart, ws, max_polls, down_only != 0, stream);
}

int i4_moe_sum(const void* res, int x_dtype, const void* ypart, const i4_moe_weights* weights,
               int topk, void* out, const void* workspace, size_t workspace_bytes,
               hipStream_t stream) {
  XBlock b;
  int rc = xblock(weights, x_dtype, topk, &b);
  if (rc) return rc;
  if (!res || !ypart || !out) return I4_ERR_NULL;
  if (((uintptr_t)res & 15) || ((uintptr_t)ypart & 15) || ((uintptr_t)out & 15))
    return I4_ERR_ALIGN;
  if (!workspace || workspace_bytes < carve(nullptr, 1, b.H, b.I, b.E, topk).bytes)
    return I4_ERR_WORKSPACE;
  if ((uintptr_t)workspace & 255) return I4_ERR_ALIGN;
  const MoeWs ws = carve(const_cast<void*>(workspace), 1, b.H, b.I, b.E, topk);
  return i4_launch_moe_sum(res, ypart, ws.w, topk, x_dtype, b.H, out, stream);
}

}  // extern "C"
