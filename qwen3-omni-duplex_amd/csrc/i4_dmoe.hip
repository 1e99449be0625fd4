// MoE block on 16-bit or int8 expert weights with an optional sigmoid-gated
// shared expert: the Talker's block.  Reference: FusedMoE.forward,
// src/duplex/streaming/fused_moe.py:99-141, which replaces transformers'
// Qwen3OmniMoeTalkerTextSparseMoeBlock (modeling_qwen3_omni_moe.py:2712-2733,
// transformers 5.15):
//   out = sum_j w_j down_e(silu(gate_e x) * up_e x)      e = sel_j, top-k of the
//                                                        router softmax, renormed
//       + sigmoid(g_s . x) * down_s(silu(gate_s x) * up_s x)   (shared expert)
// Weights: gate|up [E][2I][H] (rows [0, I) gate, [I, 2I) up: fused_moe.py:78-83)
// and down [E][H][I], either in the activation dtype or int8 with one scale per
// output row (the q8 mode, fused_moe.py:84-94: value = q * scale).
//
// Decode-shaped: the T tokens of a call run in one launch per stage (grid z / y),
// each token streaming its own experts' rows.
//   k_d_gate_up  one workgroup per (block of rows of gate and up, slot, token);
//                slot < topk is a routed expert, ranked from the logits by every
//                wave itself (workgroup (0, 0, t) also stores token t's routing);
//                slot == topk is the shared expert, whose first workgroup also
//                makes sigmoid(g_s . x).  SiLU gating happens in registers and
//                only the activation, rounded to the activation dtype as
//                fused_moe.py:127 rounds it, is written.
//   k_d_down     one output row per workgroup across every slot of one token
//                (32 lanes per slot); the routing-weighted combine, the
//                gated shared expert and an optional residual are summed in
//                fixed slot order: no atomics, bit-reproducible.
// 16-bit rows are dotted with v_dot2_f32_{f16,bf16} (exact products, fp32
// accumulation).  An int8 byte q is read as the unsigned byte q + 128 (one xor
// per word) and converted exactly to fp32; sum (q + 128) x - 128 sum x over
// each 16-byte chunk uses the chunk sums staged with the activations, and the
// row's scale multiplies the finished dot product once.
#include "i4_common.h"
#include "i4_launch.h"
#include "i4_topk.h"

namespace i4 {

static constexpr int DWG = 256;   // threads per workgroup
static constexpr int DMAXC = 8;   // 16-byte chunks of one weight row held per lane
// polls of a single-launch down workgroup before it gives up (a launch whose
// workgroups are dispatched in block order never reaches it)
static constexpr int kHandPolls = 1 << 20;

struct DW {                // one stacked weight [E][N][K]
  const void* data;        // 16-bit values, or int8 when scale != NULL
  const uint16_t* scale;   // [E][N] in the activation dtype, or NULL
  int64_t es;              // elements per expert (N * K)
  int N, K;
};

template <int XT> __device__ inline float round_to(float v) {
  return Half<XT>::to_f32(Half<XT>::from_f32(v));
}

// 16 bytes at chunk c of row n of expert e (bpe bytes per element)
__device__ inline u32x4 drow16(const DW& w, int e, int n, int c, int bpe) {
  const char* row = (const char*)w.data + ((int64_t)e * w.es + (int64_t)n * w.K) * bpe;
  return ldg16(row + 16 * (int64_t)c);
}

template <int XT> __device__ inline float dot16(u32x4 w, u32x4 x, float a) {
  a = Half<XT>::dot2(w.x, x.x, a);
  a = Half<XT>::dot2(w.y, x.y, a);
  a = Half<XT>::dot2(w.z, x.z, a);
  return Half<XT>::dot2(w.w, x.w, a);
}

// byte B of w as a float (v_cvt_f32_ubyteB)
template <int B> __device__ inline float ubyte(u32 w) { return (float)((w >> (8 * B)) & 0xFFu); }

// 16 int8 weights against xf[0..3] (the chunk's 16 activations), xsum their sum
__device__ inline float dot_i8(u32x4 w, const f32x4* xf, float xsum, float a) {
  const u32 v[4] = {w.x ^ 0x80808080u, w.y ^ 0x80808080u, w.z ^ 0x80808080u,
                    w.w ^ 0x80808080u};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f32x4 x = xf[i];
    a += ubyte<0>(v[i]) * x.x;
    a += ubyte<1>(v[i]) * x.y;
    a += ubyte<2>(v[i]) * x.z;
    a += ubyte<3>(v[i]) * x.w;
  }
  return a - 128.f * xsum;
}

// Activation staging in LDS, K values of a row (K % 16 == 0):
//   xs   [K / 8]  u32x4  the raw halves (16-bit weights)
//   xf   [K / 4]  f32x4  the values in fp32 (int8 weights only, F32)
//   xsum [K / 16] float  the sum of each 16 values (F32)
// One 8-value unit u per call; the lanes holding units u and u ^ 1 must run
// the call together (the chunk sum pairs them with a lane swizzle).
template <int XT, bool F32>
__device__ inline void commit_unit(int u, u32x4 d, u32x4* xs, f32x4* xf, float* xsum) {
  xs[u] = d;
  if constexpr (F32) {
    const u32 w[4] = {d.x, d.y, d.z, d.w};
    float f[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = Half<XT>::to_f32((uint16_t)(w[i] & 0xFFFFu));
      f[2 * i + 1] = Half<XT>::to_f32((uint16_t)(w[i] >> 16));
    }
    xf[2 * u] = f32x4{f[0], f[1], f[2], f[3]};
    xf[2 * u + 1] = f32x4{f[4], f[5], f[6], f[7]};
    const float s = ((f[0] + f[1]) + (f[2] + f[3])) + ((f[4] + f[5]) + (f[6] + f[7]));
    const float o = __builtin_bit_cast(
        float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, s), 0x041F));  // lane ^ 1
    if ((u & 1) == 0) xsum[u >> 1] = s + o;
  }
}

// byte offsets of the staging arrays for K staged values, and their total
__host__ __device__ inline size_t stage_xf_off(int K) { return (size_t)K * 2; }
__host__ __device__ inline size_t stage_xsum_off(int K) { return (size_t)K * 6; }
__host__ __device__ inline size_t stage_bytes(int K, bool f32) {
  return f32 ? (size_t)K * 6 + (size_t)K / 4 : (size_t)K * 2;
}

struct DGateUpArgs {
  const uint16_t* x;        // [T][H]
  const uint16_t* logits;   // [T][E] in the activation dtype
  int E, topk, renorm;
  int32_t* sel;             // [T][topk]
  float* wts;               // [T][topk]
  DW gu;                    // [E][2I][H]
  DW sgu;                   // [1][2Is][H]; data NULL: no shared expert
  const uint16_t* sgate_w;  // [H] or NULL (gate 1)
  float* sg;                // [T] sigmoid(g_s . x)
  uint16_t* act;            // [T][topk][I]
  uint16_t* act_s;          // [T][Is]
  int32_t* status;          // set to I4_OK by k_d_gate_up (the single launch: by the router)
};

// Expert of rank `slot` for token t; the first wave of row block 0 of slot 0
// also stores the token's sel / w.
template <int XT, int VPL>
__device__ inline int route_slot_v(const DGateUpArgs& a, int t, int bx, int slot) {
  u32 raw[VPL];
  load_row<XT, VPL>(a.logits, t, a.E, raw);
  if (bx == 0 && slot == 0 && threadIdx.x < 64) {
    int ms = 0;
    float mw = 0.f;
    topk_row<XT, VPL>(raw, t, a.E, a.topk, a.renorm, a.sel, a.wts, nullptr, 0, &ms, &mw);
    return __builtin_amdgcn_readlane(ms, 0);  // lane j holds slot j
  }
  return topk_slot<XT, VPL>(raw, a.E, slot);
}

// Rows [RPW bx, RPW (bx + 1)) of gate and up of expert e (e < 0: rank slot
// `slot` from the logits); dst[n] = silu(gate_n x) * up_n x rounded to the
// activation dtype.  COH: the values are handed to the down workgroups of the
// same launch (stored through to memory, every NaN in canonical form, so
// that no finished value looks pending).
template <int XT, bool I8, bool COH>
__device__ inline void gate_up_rows(const DGateUpArgs& a, const DW w, int e, uint16_t* dst,
                                    int t, int bx, int slot) {
  constexpr int L = I8 ? 32 : 64, RPW = DWG / L, BPE = I8 ? 1 : 2;
  const int I = w.N >> 1, H = w.K;
  if (bx * RPW >= I) return;
  extern __shared__ __align__(16) unsigned char lds[];
  u32x4* xs = (u32x4*)lds;
  f32x4* xf = (f32x4*)(lds + stage_xf_off(H));
  float* xsum = (float*)(lds + stage_xsum_off(H));
  const int units = H >> 3;  // <= DWG: one staging unit per thread
  u32x4 xd = {0u, 0u, 0u, 0u};
  if ((int)threadIdx.x < units) xd = ldg16(a.x + (int64_t)t * H + 8 * threadIdx.x);
  if (e < 0)
    e = a.E <= 128 ? route_slot_v<XT, 2>(a, t, bx, slot) : route_slot_v<XT, 8>(a, t, bx, slot);
  const int rl = threadIdx.x / L, cl = threadIdx.x % L;
  const int n = bx * RPW + rl;
  const int nn = min(n, I - 1);
  const int CH = H * BPE / 16;
  u32x4 cg[DMAXC], cu[DMAXC];
#pragma unroll
  for (int i = 0; i < DMAXC; ++i)
    if (i * L < CH) {
      const int c = min(cl + i * L, CH - 1);
      cg[i] = drow16(w, e, nn, c, BPE);
      cu[i] = drow16(w, e, I + nn, c, BPE);
    }
  if ((int)threadIdx.x < units) commit_unit<XT, I8>(threadIdx.x, xd, xs, xf, xsum);
  __syncthreads();
  float g = 0.f, u = 0.f;
#pragma unroll
  for (int i = 0; i < DMAXC; ++i) {
    const int c = cl + i * L;
    if (i * L < CH && c < CH) {
      if constexpr (I8) {
        g = dot_i8(cg[i], xf + 4 * c, xsum[c], g);
        u = dot_i8(cu[i], xf + 4 * c, xsum[c], u);
      } else {
        g = dot16<XT>(cg[i], xs[c], g);
        u = dot16<XT>(cu[i], xs[c], u);
      }
    }
  }
  g = group_sum<L>(g);
  u = group_sum<L>(u);
  // COH: the workgroup's RPW values are gathered in LDS and written through as one
  // 8- or 16-byte store (one store per value reached the pollers later, measured on
  // the Thinker's decode layer)
  __shared__ __align__(16) uint16_t s_act[RPW];
  if (cl == 0 && n < I) {
    if constexpr (I8) {
      g *= Half<XT>::to_f32(w.scale[(int64_t)e * w.N + n]);
      u *= Half<XT>::to_f32(w.scale[(int64_t)e * w.N + I + n]);
    }
    const float v = silu(g) * u;
    if constexpr (COH) s_act[rl] = v != v ? Half<XT>::QNAN : Half<XT>::from_f32(v);
    else dst[n] = Half<XT>::from_f32(v);
  }
  if constexpr (COH) {
    static_assert(RPW == 4 || RPW == 8, "8 or 16 bytes of values per workgroup");
    __syncthreads();
    const int n0 = bx * RPW, nv = min(RPW, I - n0);
    if (nv == RPW && (I & 7) == 0) {  // aligned whole store
      if (threadIdx.x == 0) {
        if constexpr (RPW == 8) {
          const rsrc_t r = rsrc(dst + n0, 16u);
          __builtin_amdgcn_raw_buffer_store_b128(*(const u32x4*)s_act, r, 0u, 0, kCoherent);
        } else {
          __hip_atomic_store((uint64_t*)(dst + n0), *(const uint64_t*)s_act, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    } else if ((int)threadIdx.x < nv) {
      st_coherent(dst + n0 + threadIdx.x, s_act[threadIdx.x]);
    }
  }
}

// sigmoid(g_s . x) of token row xr (H values), the dot product and the sigmoid
// each rounded to the activation dtype as the reference's 16-bit Linear and
// sigmoid round them (fused_moe.py:139); 1 without a gate.  Every thread of
// the workgroup calls it and receives the value.
template <int XT>
__device__ inline float shared_gate_value(const uint16_t* sgate_w, const uint16_t* xr, int H) {
  __shared__ float s_d[DWG / 64];
  if (!sgate_w) return 1.f;
  float d = 0.f;
  for (int k = threadIdx.x; k < H; k += DWG)
    d += Half<XT>::to_f32(sgate_w[k]) * Half<XT>::to_f32(xr[k]);
  d = group_sum<64>(d);
  if ((threadIdx.x & 63) == 0) s_d[threadIdx.x >> 6] = d;
  __syncthreads();
  const float z = round_to<XT>((s_d[0] + s_d[1]) + (s_d[2] + s_d[3]));
  return round_to<XT>(1.f / (1.f + expf(-z)));
}

// grid (row blocks, topk + 1, T); RI8 / SI8: routed / shared weights are int8
// one (row block bx, slot) of token t's gate|up stage
template <int XT, bool RI8, bool SI8, bool COH>
__device__ inline void d_gate_up_block(const DGateUpArgs& a, int bx, int slot, int t) {
  if (slot < a.topk) {
    gate_up_rows<XT, RI8, COH>(a, a.gu, -1, a.act + ((int64_t)t * a.topk + slot) * (a.gu.N >> 1),
                               t, bx, slot);
  } else if (a.sgu.data) {
    gate_up_rows<XT, SI8, COH>(a, a.sgu, 0, a.act_s + (int64_t)t * (a.sgu.N >> 1), t, bx, slot);
  }
}

template <int XT, bool RI8, bool SI8>
__global__ __launch_bounds__(DWG) void k_d_gate_up(DGateUpArgs a) {
  const int t = blockIdx.z, slot = blockIdx.y;
  if (a.status && (blockIdx.x | blockIdx.y | blockIdx.z | threadIdx.x) == 0) *a.status = I4_OK;
  d_gate_up_block<XT, RI8, SI8, false>(a, blockIdx.x, slot, t);
  if (slot == a.topk && a.sgu.data && blockIdx.x == 0) {
    const float g = shared_gate_value<XT>(a.sgate_w, a.x + (int64_t)t * a.sgu.K, a.sgu.K);
    if (threadIdx.x == 0) a.sg[t] = g;
  }
}

struct DDownArgs {
  const uint16_t* act;       // [T][topk][I]
  const uint16_t* act_s;     // [T][Is]
  int topk;
  const int32_t* sel;        // [T][topk]
  const float* wts;          // [T][topk]
  const float* sg;           // [T]
  DW dn;                     // [E][H][I]
  DW sdn;                    // [1][H][Is]; data NULL: no shared expert
  const uint16_t* residual;  // [T][H] or NULL
  uint16_t* out;             // [T][H]
};

// What the down workgroups of a single-launch decode (k_d_moe1) derive
// themselves instead of reading it from the gate|up launch: the experts and
// routing weights (ranked from the logits, bit-identical to the gate|up
// workgroups) and the shared gate; act / act_s they poll as it is written.
struct DHand {
  const uint16_t* logits;   // [T][E]
  int E, renorm;
  const uint16_t* x;        // [T][H]
  const uint16_t* sgate_w;  // [H] or NULL
  int max_polls;
  int32_t* status;          // set to I4_ERR_HANDOFF by a workgroup that gave up
};

// Row bx of token t.  Lane group g (32 lanes) computes row bx of slot g
// (slot topk: the shared expert; higher slots idle).  Lane counts here and in
// the gate|up stage (one wave per 16-bit row pair, half a wave per int8 pair)
// were picked by a sweep at the Talker's shapes: within 0.5 us of each other
// per block for bf16, 1 us faster than half as many lanes for int8.
// HANDOFF: see DHand; the staged activations are polled (at most 2 DWG
// 16-byte units, checked by the host) until none holds the pending pattern.
template <int XT, bool RI8, bool SI8, bool HANDOFF, int RW>
__device__ inline void d_down_rows(const DDownArgs& a, int bx, int t, const DHand& h) {
  constexpr int L = 32, NSG = 8;
  constexpr bool F32 = RI8 || SI8;
  const int topk = a.topk;
  const int I = a.dn.K, H = a.dn.N;
  const int Is = a.sdn.data ? a.sdn.K : 0;
  const int KR = topk * I, KT = KR + Is;
  extern __shared__ __align__(16) unsigned char lds[];
  u32x4* xs = (u32x4*)lds;
  f32x4* xf = (f32x4*)(lds + stage_xf_off(KT));
  float* xsum = (float*)(lds + stage_xsum_off(KT));
  __shared__ float red[RW][NSG];
  __shared__ float s_w[NSG];  // HANDOFF: the routing weights
  const int grp = threadIdx.x / L, cl = threadIdx.x % L;
  const int j = grp % NSG;
  const bool sh = Is > 0 && j == topk;
  const bool live = j < topk || sh;
  int e = 0;
  if constexpr (HANDOFF) {
    // every wave ranks the token's logits; lane s < topk holds slot s
    int ms = 0;
    float mw = 0.f;
    if (h.E <= 128) {
      u32 raw[2];
      load_row<XT, 2>(h.logits, t, h.E, raw);
      topk_row<XT, 2>(raw, t, h.E, topk, h.renorm, nullptr, nullptr, nullptr, 0, &ms, &mw);
    } else {
      u32 raw[8];
      load_row<XT, 8>(h.logits, t, h.E, raw);
      topk_row<XT, 8>(raw, t, h.E, topk, h.renorm, nullptr, nullptr, nullptr, 0, &ms, &mw);
    }
    // every lane takes part in the shuffle; the shared slot reads expert 0 of
    // its one-expert stack, idle slots nothing
    const int ej = __shfl(ms, j < topk ? j : 0, 64);
    e = j < topk ? ej : 0;
    if ((int)threadIdx.x < topk) s_w[threadIdx.x] = mw;
  } else {
    e = j < topk ? a.sel[(int64_t)t * topk + j] : 0;
  }
  const DW w = sh ? a.sdn : a.dn;
  const bool i8 = sh ? SI8 : RI8;
  const int CH = i8 ? w.K / 16 : w.K / 8;
  u32x4 cw[RW][DMAXC];
  if (live) {
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int nn = min(bx * RW + r, H - 1);
#pragma unroll
      for (int i = 0; i < DMAXC; ++i)
        if (i * L < CH) cw[r][i] = drow16(w, e, nn, min(cl + i * L, CH - 1), i8 ? 1 : 2);
    }
  }
  // stage the token's activations: the routed slots, then the shared one
  const int units = KT >> 3, ur = KR >> 3;
  bool late = false;
  float sg = 0.f;
  if constexpr (HANDOFF) {
    if (Is > 0) sg = shared_gate_value<XT>(h.sgate_w, h.x + (int64_t)t * a.sdn.N, a.sdn.N);
    const rsrc_t ra = rsrc(a.act + (int64_t)t * KR, (u32)KR * 2u);
    const rsrc_t rs = rsrc(a.act_s + (int64_t)t * Is, (u32)Is * 2u);
    u32x4 d[2];
    for (int it = 0;; ++it) {
      bool pend = false;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int u = (int)threadIdx.x + q * DWG;
        if (u < units) {
          d[q] = u < ur ? ld16_coherent(ra, (u32)u * 16u) : ld16_coherent(rs, (u32)(u - ur) * 16u);
          pend |= has_pending(d[q]);
        }
      }
      if (!__syncthreads_or(pend)) break;
      if (it >= h.max_polls) {
        late = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int u = (int)threadIdx.x + q * DWG;
      if (u < units) commit_unit<XT, F32>(u, d[q], xs, xf, xsum);
    }
  } else {
    for (int u = threadIdx.x; u < units; u += DWG) {
      const u32x4 d = u < ur ? ldg16(a.act + (int64_t)t * KR + 8 * u)
                             : ldg16(a.act_s + (int64_t)t * Is + 8 * (u - ur));
      commit_unit<XT, F32>(u, d, xs, xf, xsum);
    }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    float acc = 0.f;
    if (live) {
      const int base = j < topk ? j * I : KR;  // staged offset of this slot's row
      if (i8) {
#pragma unroll
        for (int i = 0; i < DMAXC; ++i) {
          const int c = cl + i * L;
          if (i * L < CH && c < CH)
            acc = dot_i8(cw[r][i], xf + (base >> 2) + 4 * c, xsum[(base >> 4) + c], acc);
        }
      } else {
#pragma unroll
        for (int i = 0; i < DMAXC; ++i) {
          const int c = cl + i * L;
          if (i * L < CH && c < CH) acc = dot16<XT>(cw[r][i], xs[(base >> 3) + c], acc);
        }
      }
    }
    acc = group_sum<L>(acc);
    if (cl == 0) {
      if (live && i8) acc *= Half<XT>::to_f32(w.scale[(int64_t)e * w.N + min(bx * RW + r, H - 1)]);
      red[r][j] = acc;
    }
  }
  __syncthreads();
  const int row = bx * RW + (int)threadIdx.x;
  if ((int)threadIdx.x < RW && row < H) {
    float y = 0.f;
    for (int s = 0; s < topk; ++s)
      y += (HANDOFF ? s_w[s] : a.wts[(int64_t)t * topk + s]) * red[threadIdx.x][s];
    if (Is > 0) y += (HANDOFF ? sg : a.sg[t]) * red[threadIdx.x][topk];
    if (a.residual) y += Half<XT>::to_f32(a.residual[(int64_t)t * H + row]);
    if (late) y = __builtin_nanf("");
    a.out[(int64_t)t * H + row] = Half<XT>::from_f32(y);
  }
  if constexpr (HANDOFF) {
    if (late && threadIdx.x == 0) *h.status = I4_ERR_HANDOFF;
  }
}

// grid (H, T)
template <int XT, bool RI8, bool SI8>
__global__ __launch_bounds__(DWG) void k_d_down(DDownArgs a) {
  d_down_rows<XT, RI8, SI8, false, 1>(a, blockIdx.x, blockIdx.y, DHand{});
}

// output rows per down workgroup of k_d_moe1: with 2 the 512 down workgroups
// start beside the 1344 gate|up ones instead of waiting for their slots (1:
// 14.9 us per Talker block, 2: 13.05 us, 4 and 8: 16.3 and 23.1 us, their
// weight registers spilling)
static constexpr int DRW1 = 2;

// One decode token (T = 1) whose router ran in the launch before, both stages
// in one launch: blocks [0, gx (topk + 1)) are the gate|up blocks (row block,
// slot), blocks from n_gu on the H down rows.  The router launch fills act and
// act_s with the pending pattern; the gate|up blocks, dispatched first,
// overwrite every value.  n_gu = 0: the down rows alone (the activations are
// then never written, and every down block gives up after max_polls polls).
template <int XT, bool RI8, bool SI8>
__global__ __launch_bounds__(DWG) void k_d_moe1(DGateUpArgs a, DDownArgs d, DHand h, int gx,
                                                int n_gu) {
  const int b = blockIdx.x;
  if (b < n_gu) d_gate_up_block<XT, RI8, SI8, true>(a, b % gx, b / gx, 0);
  else d_down_rows<XT, RI8, SI8, true, DRW1>(d, b - n_gu, 0, h);
}

}  // namespace i4

using namespace i4;

namespace {

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

struct DmoeWs {
  size_t logits, sel, wts, sg, status, act, act_s, total;
};

// act_s follows act directly: the router launch of a single-launch decode
// marks both pending as one range
DmoeWs dmoe_ws_layout(int T, int E, int topk, int I, int Is) {
  DmoeWs l;
  size_t o = 0;
  l.logits = o; o += align256((size_t)T * E * 2);
  l.sel = o;    o += align256((size_t)T * topk * 4);
  l.wts = o;    o += align256((size_t)T * topk * 4);
  l.sg = o;     o += align256((size_t)T * 4);
  l.status = o; o += align256(4);
  l.act = o;    o += align256((size_t)T * topk * I * 2);
  l.act_s = o;  o += align256((size_t)T * Is * 2);
  l.total = o;
  return l;
}

// the single launch stages at most two 16-byte units per thread
bool dmoe1_fits(int topk, int I, int Is) { return (topk * I + Is) / 8 <= 2 * DWG; }

// 16-byte chunks of one row of K elements (int8 rows: 16 values, 16-bit: 8)
int row_chunks(const i4_dweight& w, int K) { return w.scale ? K / 16 : K / 8; }

int check_dweight(const i4_dweight& w, int E, int N, int K) {
  if (!w.data) return I4_ERR_NULL;
  if ((uintptr_t)w.data & 15) return I4_ERR_ALIGN;
  if ((uintptr_t)w.scale & 1) return I4_ERR_ALIGN;
  if (w.E != E || w.N != N || w.K != K) return I4_ERR_SHAPE;
  return I4_OK;
}

DW to_dw(const i4_dweight& w) {
  DW d;
  d.data = w.data;
  d.scale = (const uint16_t*)w.scale;
  d.es = (int64_t)w.N * w.K;
  d.N = w.N;
  d.K = w.K;
  return d;
}

// hand: T = 1 in one launch (k_d_moe1), act / act_s marked pending by the
// router launch before it; gate_up = false runs its down blocks alone
template <int XT, bool RI8, bool SI8>
int dmoe_launch(const DGateUpArgs& ga, const DDownArgs& da, int T, int H, const DHand* hand,
                bool gate_up, hipStream_t s) {
  const int I = ga.gu.N >> 1, Is = ga.sgu.data ? ga.sgu.N >> 1 : 0;
  const int rpw_r = RI8 ? DWG / 32 : DWG / 64, rpw_s = SI8 ? DWG / 32 : DWG / 64;
  const int bx = max((I + rpw_r - 1) / rpw_r, Is ? (Is + rpw_s - 1) / rpw_s : 0);
  const size_t lds = max(stage_bytes(H, RI8 || SI8), stage_bytes(da.topk * I + Is, RI8 || SI8));
  if (hand) {
    const int n_gu = gate_up ? bx * (ga.topk + 1) : 0;
    hipLaunchKernelGGL((k_d_moe1<XT, RI8, SI8>), dim3(n_gu + (H + DRW1 - 1) / DRW1), dim3(DWG),
                       lds, s, ga, da, *hand, bx, n_gu);
    return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;
  }
  hipLaunchKernelGGL((k_d_gate_up<XT, RI8, SI8>), dim3(bx, ga.topk + 1, T), dim3(DWG),
                     stage_bytes(H, RI8 || SI8), s, ga);
  if (hipGetLastError() != hipSuccess) return I4_ERR_LAUNCH;
  hipLaunchKernelGGL((k_d_down<XT, RI8, SI8>), dim3(H, T), dim3(DWG),
                     stage_bytes(da.topk * I + Is, RI8 || SI8), s, da);
  return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;
}

}  // namespace

extern "C" size_t i4_dmoe_workspace_bytes(int T, int E, int topk, int I, int Is) {
  if (T < 1 || E < 1 || topk < 1 || I < 0 || Is < 0) return 0;
  return dmoe_ws_layout(T, E, topk, I, Is).total;
}

namespace {

// i4_dmoe_forward, or (down_wait) the down stage of the single launch alone
// with max_polls as its bound, on the workspace's activations as they are
int dmoe_impl(const void* x, int x_dtype, int T, const i4_dmoe_weights* wts, int topk,
              int renorm, const void* logits, const void* residual, void* out, int32_t* sel_out,
              float* w_out, void* workspace, size_t workspace_bytes, bool down_wait,
              int max_polls, hipStream_t stream) {
  if (!x || !wts || !out) return I4_ERR_NULL;
  if (!wts->router_w && !logits) return I4_ERR_NULL;
  if (x_dtype != I4_F16 && x_dtype != I4_BF16) return I4_ERR_DTYPE;
  const i4_dweight& gu = wts->gate_up;
  const i4_dweight& dn = wts->down;
  const int E = gu.E, I = gu.N / 2, H = gu.K;
  const bool has_shared = wts->shared_gate_up.data != nullptr;
  if (T < 1 || T > 65535 || E < 1 || E > 512 || H < 16 || H > 2048 || H % 16 || I < 16 ||
      I % 16 || gu.N != 2 * I || topk < 1 || topk > E || topk > (has_shared ? 7 : 8))
    return I4_ERR_SHAPE;
  int rc = check_dweight(gu, E, 2 * I, H);
  if (rc == I4_OK) rc = check_dweight(dn, E, H, I);
  if (rc != I4_OK) return rc;
  if (!gu.scale != !dn.scale) return I4_ERR_DTYPE;  // routed experts: one format
  if (row_chunks(dn, I) > DMAXC * 16) return I4_ERR_SHAPE;
  int Is = 0;
  if (has_shared) {
    const i4_dweight& sgu = wts->shared_gate_up;
    const i4_dweight& sdn = wts->shared_down;
    Is = sgu.N / 2;
    if (Is < 16 || Is % 16 || sgu.N != 2 * Is) return I4_ERR_SHAPE;
    rc = check_dweight(sgu, 1, 2 * Is, H);
    if (rc == I4_OK) rc = check_dweight(sdn, 1, H, Is);
    if (rc != I4_OK) return rc;
    if (!sgu.scale != !sdn.scale) return I4_ERR_DTYPE;
    if (row_chunks(sdn, Is) > DMAXC * 16) return I4_ERR_SHAPE;
    if ((uintptr_t)wts->shared_gate_w & 1) return I4_ERR_ALIGN;
  } else if (wts->shared_down.data || wts->shared_gate_w) {
    return I4_ERR_NULL;  // shared down or gate given without the shared gate|up
  }
  if (((uintptr_t)x & 15) || ((uintptr_t)out & 15) || ((uintptr_t)residual & 15) ||
      ((uintptr_t)wts->router_w & 15) || ((uintptr_t)logits & 1))
    return I4_ERR_ALIGN;
  const bool ri8 = gu.scale != nullptr, si8 = has_shared && wts->shared_gate_up.scale;
  if (stage_bytes(topk * I + Is, ri8 || si8) > 65536) return I4_ERR_SHAPE;
  const DmoeWs l = dmoe_ws_layout(T, E, topk, I, Is);
  if (!workspace || workspace_bytes < l.total) return I4_ERR_WORKSPACE;
  if ((uintptr_t)workspace & 15) return I4_ERR_ALIGN;
  char* ws = (char*)workspace;
  int32_t* status = (int32_t*)(ws + l.status);
  // one token with the router in the block and 16-bit routed experts: gate|up
  // and down in one launch whose down workgroups wait for the activations (the
  // router launch marks them pending first).  Measured per Talker block against
  // three launches on one box: bf16 13.05 vs 13.07 us, int8 12.67 vs 12.41 us,
  // so int8 experts keep three launches.
  const bool one = T == 1 && wts->router_w && !ri8 && dmoe1_fits(topk, I, Is);
  if (down_wait) {
    if (T != 1 || !logits || !dmoe1_fits(topk, I, Is)) return I4_ERR_SHAPE;
    if (ri8) return I4_ERR_DTYPE;  // the single launch serves 16-bit routed experts
    if (max_polls < 0) return I4_ERR_SHAPE;
  }
  const void* lg = logits;
  if (wts->router_w && !down_wait) {
    lg = ws + l.logits;
    rc = i4_launch_router_logits(x, x_dtype, T, H, wts->router_w, E, nullptr, 0.f, nullptr,
                                 (void*)lg, stream, one ? ws + l.act : nullptr,
                                 one ? (int)((l.act_s - l.act + (size_t)Is * 2) / 16) : 0,
                                 one ? status : nullptr);
    if (rc != I4_OK) return rc;
  }
  DGateUpArgs ga;
  ga.x = (const uint16_t*)x;
  ga.logits = (const uint16_t*)lg;
  ga.E = E;
  ga.topk = topk;
  ga.renorm = renorm;
  ga.sel = sel_out ? sel_out : (int32_t*)(ws + l.sel);
  ga.wts = w_out ? w_out : (float*)(ws + l.wts);
  ga.gu = to_dw(gu);
  ga.sgu = has_shared ? to_dw(wts->shared_gate_up) : DW{nullptr, nullptr, 0, 0, 0};
  ga.sgate_w = (const uint16_t*)wts->shared_gate_w;
  ga.sg = (float*)(ws + l.sg);
  ga.act = (uint16_t*)(ws + l.act);
  ga.act_s = (uint16_t*)(ws + l.act_s);
  ga.status = status;
  DDownArgs da;
  da.act = ga.act;
  da.act_s = ga.act_s;
  da.topk = topk;
  da.sel = ga.sel;
  da.wts = ga.wts;
  da.sg = ga.sg;
  da.dn = to_dw(dn);
  da.sdn = has_shared ? to_dw(wts->shared_down) : DW{nullptr, nullptr, 0, 0, 0};
  da.residual = (const uint16_t*)residual;
  da.out = (uint16_t*)out;
  const DHand hand{(const uint16_t*)lg, E, renorm, (const uint16_t*)x, ga.sgate_w,
                   down_wait ? max_polls : kHandPolls, status};
  const DHand* hp = one || down_wait ? &hand : nullptr;
#define I4_DMOE_CASE(XT_, R_, S_)                                                                \
  if (x_dtype == XT_ && ri8 == R_ && si8 == S_)                                                  \
    return dmoe_launch<XT_, R_, S_>(ga, da, T, H, hp, !down_wait, stream);
  I4_DMOE_CASE(I4_F16, false, false)
  I4_DMOE_CASE(I4_F16, true, false)
  I4_DMOE_CASE(I4_F16, true, true)
  I4_DMOE_CASE(I4_F16, false, true)
  I4_DMOE_CASE(I4_BF16, false, false)
  I4_DMOE_CASE(I4_BF16, true, false)
  I4_DMOE_CASE(I4_BF16, true, true)
  I4_DMOE_CASE(I4_BF16, false, true)
#undef I4_DMOE_CASE
  return I4_ERR_DTYPE;
}

}  // namespace

extern "C" int i4_dmoe_forward(const void* x, int x_dtype, int T, const i4_dmoe_weights* wts,
                               int topk, int renorm, const void* logits, const void* residual,
                               void* out, int32_t* sel_out, float* w_out, void* workspace,
                               size_t workspace_bytes, hipStream_t stream) {
  return dmoe_impl(x, x_dtype, T, wts, topk, renorm, logits, residual, out, sel_out, w_out,
                   workspace, workspace_bytes, false, 0, stream);
}

extern "C" size_t i4_dmoe_status_offset(int T, int E, int topk, int I, int Is) {
  if (T < 1 || E < 1 || topk < 1 || I < 0 || Is < 0) return 0;
  return dmoe_ws_layout(T, E, topk, I, Is).status;
}

extern "C" int i4_dmoe_down_wait(const void* x, int x_dtype, const i4_dmoe_weights* wts,
                                 int topk, int renorm, const void* logits, const void* residual,
                                 void* out, void* workspace, size_t workspace_bytes,
                                 int max_polls, hipStream_t stream) {
  return dmoe_impl(x, x_dtype, 1, wts, topk, renorm, logits, residual, out, nullptr, nullptr,
                   workspace, workspace_bytes, true, max_polls, stream);
}
