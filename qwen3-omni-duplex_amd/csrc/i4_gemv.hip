// int4 dequant-GEMV kernels for gfx950 and their C-ABI entry points.
//
//   k_gemv_ct      gathered GEMV on the compressed-tensors layout
//                  (replaces _dq_gemv_kernel, triton_dequant_gemv.py:32-82)
//   k_gemv_awq     GEMV straight on AutoAWQ packing, one launch (K reduced
//                  inside each workgroup)
//   k_unpack       raw nibbles in logical [E][N][K] order (unpack4,
//                  fused_packed_moe.py:54-65)
//   k_dequant      dense (q - z) * s (FusedPackedMoE._dequant, :183-189)
//   k_repack_awq   AWQ -> CT(+zeros) conversion done once at load time
//
// The CT GEMV's work split is described with its body (i4_gemv_body.h); grid.y
// is the selected-expert slot.
#include <atomic>

#include "i4_common.h"
#include "i4_gemv_body.h"
#include "i4_launch.h"
#include "i4_moe_launch.h"

namespace i4 {

static constexpr int WG = GEMV_WG;

template <int XT, int ST, int L, bool NORM>
__global__ __launch_bounds__(WG) void k_gemv_ct(
    const uint16_t* __restrict__ x, int64_t x_stride, const int32_t* __restrict__ packed,
    int64_t p_es, const void* __restrict__ scale, int64_t s_es,
    const int32_t* __restrict__ zeros, int64_t z_es, const int32_t* __restrict__ sel, int E,
    int N, int K, int gshift, void* __restrict__ out, int ot, const void* __restrict__ bias,
    const uint16_t* __restrict__ nw, float eps) {
  extern __shared__ __align__(16) unsigned char lds[];
  gemv_ct_body<XT, ST, L, NORM, false>(blockIdx.x, blockIdx.y, x, x_stride, packed, p_es, scale,
                                       s_es, zeros, z_es, sel, E, N, K, gshift, out, ot, bias,
                                       nw, eps, lds, 0);
}

// ---------------------------------------------------------------------------
// AWQ GEMV in one launch.  A workgroup owns one column word (8 output columns)
// of one selected expert over all of K, so the K reduction stays inside it and
// the launch has N / 8 workgroups per expert: thread t takes the row blocks t,
// t + 256, ... of RB rows (RB divides the group, so a block lies in one
// quantisation group).  Row pairs (k, k+1) of a column are merged byte-wise
// with v_perm_b32 into (M + q_k, M + q_k+1) halves for v_dot2 against (x_k,
// x_k+1); per block and column the bias M and the zero point are removed with
// the block's activation sum and the block's scale applied:
//     s (sum (M + q) x - (M + z) sum x).
// The 256 partials of a column are then summed in a fixed order (wave sums,
// then the four waves), so the result does not depend on timing.  Measured
// on the 2048 -> 768 GEMV: one word per workgroup beats two or four (which
// halve / quarter the workgroups: 12.5 / 13.6 us against 6.2), and the
// XCD-aware tile order below beats plain block order (6.6 -> 6.2 us; q_proj
// 2048 -> 4096 11.3 -> 8.8 us).
__device__ inline constexpr int awq_col(int slot) {  // column of nibble slot, 0,2,4,6,1,3,5,7
  return (slot & 3) * 2 + (slot >> 2);
}

template <int XT, int ST, int RB>
__global__ __launch_bounds__(WG) void k_gemv_awq(
    const uint16_t* __restrict__ x, int64_t x_stride, const int32_t* __restrict__ qw, int64_t q_es,
    const void* __restrict__ scales, int64_t s_es, const int32_t* __restrict__ qz, int64_t z_es,
    const int32_t* __restrict__ sel, int E, int N, int K, int gshift, void* __restrict__ out,
    int ot, const void* __restrict__ bias) {
  __shared__ float red[WG / 64][8];
  const int NW = N >> 3;
  // XCD-aware word order: workgroups are dispatched round-robin over the 8 XCDs
  // (block b on XCD b % 8), so each XCD gets a contiguous run of words and the
  // words that share a cache line are mostly read through one XCD's L2
  int cw = blockIdx.x;
  const int per = (int)gridDim.x >> 3;
  if ((int)blockIdx.x < per * 8) cw = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
  const int j = blockIdx.y;
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const int e = sel ? sel[j] : 0;
  const bool ev = (unsigned)e < (unsigned)E;
  const int ee = ev ? e : 0;
  const int32_t* qe = qw + ee * q_es + cw;
  const int32_t* ze = qz ? qz + ee * z_es + cw : nullptr;
  const uint16_t* xrow = x + (int64_t)j * x_stride;
  constexpr u32 MK = 0x000F000Fu;
  const u32 mg = magic_v<XT>();
  const u32 ONE2 = XT == I4_F16 ? 0x3C003C00u : 0x3F803F80u;  // (1.0, 1.0)
  constexpr int SPL = ST == I4_F32 ? 4 : 8;  // scales per 16-byte load
  float tot[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) tot[c] = 0.f;
  for (int k0 = t * RB; k0 < K; k0 += WG * RB) {
    // every load of the block first: weights, activations, scales, zero word
    u32 wv[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) wv[r] = (u32)qe[(int64_t)(k0 + r) * NW];
    u32 xp[RB / 2];
#pragma unroll
    for (int p = 0; p < RB / 2; ++p) xp[p] = *(const u32*)(xrow + k0 + 2 * p);
    const int g = k0 >> gshift;
    const char* sp = (const char*)scales + (ee * s_es + (int64_t)g * N + 8 * cw) *
                                               (ST == I4_F32 ? 4 : 2);
    u32x4 sv[8 / SPL];
#pragma unroll
    for (int v = 0; v < 8 / SPL; ++v) sv[v] = ldg16(sp + 16 * v);
    const u32 zw = ze ? (u32)ze[(int64_t)g * NW] : 0x88888888u;
    float acc[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] = 0.f;
    float S = 0.f;
#pragma unroll
    for (int p = 0; p < RB / 2; ++p) {
      S = Half<XT>::dot2(xp[p], ONE2, S);
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        // byte b of row 2p -> bits 0..7, byte b of row 2p + 1 -> bits 16..23
        const u32 sel_b = 0x0C000C00u | (u32)(b) | ((u32)(4 + b) << 16);
        const u32 tb = __builtin_amdgcn_perm(wv[2 * p + 1], wv[2 * p], sel_b);
        acc[2 * b] = Half<XT>::dot2((tb & MK) | mg, xp[p], acc[2 * b]);
        acc[2 * b + 1] = Half<XT>::dot2(((tb >> 4) & MK) | mg, xp[p], acc[2 * b + 1]);
      }
    }
#pragma unroll
    for (int sl = 0; sl < 8; ++sl) {
      const float z = (float)((zw >> (4 * sl)) & 15u);
      const int c = awq_col(sl);
      const u32x4 q = sv[c / SPL];
      const int ci = c % SPL;
      const int wsel = ST == I4_F32 ? ci : ci >> 1;
      const u32 word = wsel == 0 ? q.x : wsel == 1 ? q.y : wsel == 2 ? q.z : q.w;
      const u32 raw = ST == I4_F32 ? word : (ci & 1 ? word >> 16 : word & 0xFFFFu);
      tot[sl] += scale_from_raw<ST>(raw) * (acc[sl] - (Half<XT>::MAGIC + z) * S);
    }
  }
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const float v = group_sum<64>(tot[c]);
    if (lane == 0) red[wave][c] = v;
  }
  __syncthreads();
  if (t < 8) {
    float v = ((red[0][t] + red[1][t]) + red[2][t]) + red[3][t];
    if (!ev) v = __builtin_nanf("");
    const int n = 8 * cw + awq_col(t);
    const int64_t o = (int64_t)j * N + n;
    if (ot == I4_F32) {
      if (bias) v += ((const float*)bias)[n];
      store_out<I4_F32>(out, o, v);
    } else if (ot == I4_F16) {
      if (bias) v += Half<I4_F16>::to_f32(((const uint16_t*)bias)[n]);
      store_out<I4_F16>(out, o, v);
    } else {
      if (bias) v += Half<I4_BF16>::to_f32(((const uint16_t*)bias)[n]);
      store_out<I4_BF16>(out, o, v);
    }
  }
}

// ---------------------------------------------------------------------------
// AWQ GEMV split along K, one launch.  A K-complete workgroup reads a column
// word as 4 bytes out of every 128-byte line of its K rows, so each CU fills
// K lines for 4 K bytes of weights (2048-4096 fills per CU at the attention
// shapes).  Here a workgroup owns a strip of 256 columns (32 words: one whole
// line per row) over a slice of KS rows, so every line it fills is used in
// full and the launch has (N / 256) x (K / KS) workgroups per row of x:
//   thread t: quad q = t & 7 (words 4q..4q+3 of the strip, 32 columns) and
//   row pair rp = t >> 3 of each 16 * NWAVE-row pass (rows k, k+1 merged
//   byte-wise into (M + q_k, M + q_k+1) halves for v_dot2, as in k_gemv_awq);
//   the zero point is removed per thread with its pair sums of x, the
//   per-thread column sums are reduced over the row pairs with a halving lane
//   butterfly (xor 8, 16, 32: each step keeps half the columns) and then
//   across the waves in LDS, and the slice's scale (loaded with the weights)
//   is applied once per column: a slice lies inside one quantisation group.
// Hand-over without atomics or fences, inside one XCD: every slice of a strip runs on
// the same XCD, slices 0..P-2 store their fp32 partials (1 KB) into that XCD's L2 and
// exit, each column as one 8-byte store of (value, tag) with the call's tag (a number
// the host gives every call, never 0); slice P-1, dispatched after them, reads the
// other partials past its L1 (from the L2 that holds them) until every one carries the
// call's tag, sums them in a fixed order (slice classes s mod NWAVE, then its own
// slice), writes y, and clears the tags it read (so a captured graph, which replays one
// tag, finds them pending again).  A partial left by an earlier
// call never carries this call's tag, so the workspace needs no initial contents.
// A reducer that polls max_polls times without seeing every partial writes NaN,
// clears the tags of its whole strip and stores I4_ERR_HANDOFF in the status word
// (the workspace's first int32; only failures are stored, the caller clears it).
static constexpr int SK_COLS = 256;  // columns per strip
static constexpr int kAwqPolls = 1 << 20;
static constexpr size_t SK_HEAD = 256;  // workspace header: the status word, then partials

template <int XT, int ST, int NWAVE, int PPT>
__global__ __launch_bounds__(64 * NWAVE) void k_gemv_awq_sk(
    const uint16_t* __restrict__ x, int64_t x_stride, const int32_t* __restrict__ qw, int64_t q_es,
    const void* __restrict__ scales, int64_t s_es, const int32_t* __restrict__ qz, int64_t z_es,
    const int32_t* __restrict__ sel, int E, int N, int gshift, int S, int P,
    uint64_t* part, void* __restrict__ out, int ot, const void* __restrict__ bias, int max_polls,
    u32 tag, int32_t* __restrict__ status, int only_last) {
  constexpr int NT = 64 * NWAVE, PASS = 16 * NWAVE, KS = PASS * PPT, CPT = SK_COLS / NT;
  __shared__ f32x4 red[NWAVE][64];
  __shared__ int s_gave_up;  // the reducer's wait gave up (set before the first barrier)
  // only_last: the reducers alone (grid S), whose partials then never arrive -- the host's
  // way of making the wait give up in a test.  Otherwise every slice of a strip runs on
  // one XCD (block b on XCD b % 8; strip x + 8 l takes the P blocks b = 8 (l P + slice)
  // + x, past S: none), so the partials are handed over through that XCD's L2
  int strip, slice;
  if (only_last) {
    strip = (int)blockIdx.x;
    slice = P - 1;
  } else {
    const int i = (int)blockIdx.x >> 3;
    strip = ((int)blockIdx.x & 7) + 8 * (i / P);
    slice = i % P;
    if (strip >= S) return;
  }
  const int j = blockIdx.y;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int q = t & 7, rp = t >> 3;
  const int NW = N >> 3;
  const int e = sel ? sel[j] : 0;
  const bool ev = (unsigned)e < (unsigned)E;
  const int ee = ev ? e : 0;
  const int w0 = strip * 32 + 4 * q;  // N % 32 == 0: a quad is wholly inside or outside
  const int wc = w0 < NW ? w0 : 0;
  const int k0 = slice * KS, g = k0 >> gshift;
  const int32_t* qe = qw + ee * q_es + wc;
  const uint16_t* xrow = x + (int64_t)j * x_stride;

  // every load first: weight row pairs, x pairs, the zero words, the output
  // columns' scales (thread t finishes strip columns ct = t + NT c, mapped as
  // quad ct >> 5, word (ct >> 3) & 3 of the quad, nibble slot ct & 7)
  u32x4 wa[PPT], wb[PPT];
  u32 xp[PPT];
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    const int k = k0 + 2 * (rp + (PASS / 2) * i);
    wa[i] = ldg16(qe + (int64_t)k * NW);
    wb[i] = ldg16(qe + (int64_t)(k + 1) * NW);
  }
#pragma unroll
  for (int i = 0; i < PPT; ++i) xp[i] = *(const u32*)(xrow + k0 + 2 * (rp + (PASS / 2) * i));
  u32x4 zv = {0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};
  if (qz) zv = ldg16(qz + ee * z_es + (int64_t)g * NW + wc);
  int ncol[CPT];
  u32 sraw[CPT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int ct = t + NT * c;
    const int word = strip * 32 + (ct >> 3);
    ncol[c] = word < NW ? 8 * word + awq_col(ct & 7) : -1;
    sraw[c] = load_scale_raw<ST>(scales, ee * s_es + (int64_t)g * N + (word < NW ? ncol[c] : 0));
  }

  constexpr u32 MK = 0x000F000Fu;
  const u32 mg = magic_v<XT>();
  const u32 ONE2 = XT == I4_F16 ? 0x3C003C00u : 0x3F803F80u;  // (1.0, 1.0)
  float acc[32];  // column slot sl of word jw at 8 jw + sl
#pragma unroll
  for (int c = 0; c < 32; ++c) acc[c] = 0.f;
  float Sx = 0.f;
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    Sx = Half<XT>::dot2(xp[i], ONE2, Sx);
    const u32 av[4] = {wa[i].x, wa[i].y, wa[i].z, wa[i].w};
    const u32 bv[4] = {wb[i].x, wb[i].y, wb[i].z, wb[i].w};
#pragma unroll
    for (int jw = 0; jw < 4; ++jw) {
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        // byte b of row k -> bits 0..7, byte b of row k + 1 -> bits 16..23
        const u32 sel_b = 0x0C000C00u | (u32)(b) | ((u32)(4 + b) << 16);
        const u32 tb = __builtin_amdgcn_perm(bv[jw], av[jw], sel_b);
        acc[8 * jw + 2 * b] = Half<XT>::dot2((tb & MK) | mg, xp[i], acc[8 * jw + 2 * b]);
        acc[8 * jw + 2 * b + 1] =
            Half<XT>::dot2(((tb >> 4) & MK) | mg, xp[i], acc[8 * jw + 2 * b + 1]);
      }
    }
  }
  {
    const u32 zw[4] = {zv.x, zv.y, zv.z, zv.w};
#pragma unroll
    for (int jw = 0; jw < 4; ++jw)
#pragma unroll
      for (int sl = 0; sl < 8; ++sl)
        acc[8 * jw + sl] =
            fmaf(-(Half<XT>::MAGIC + (float)((zw[jw] >> (4 * sl)) & 15u)), Sx, acc[8 * jw + sl]);
  }

  // halving butterfly over the 8 row pairs of the wave that share q
  const bool h1 = (lane >> 3) & 1, h2 = (lane >> 4) & 1, h3 = (lane >> 5) & 1;
  float u1[16], u2[8];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float keep = h1 ? acc[16 + i] : acc[i], send = h1 ? acc[i] : acc[16 + i];
    u1[i] = keep + dpp_mov<0x128>(send);  // row_ror:8, lane ^ 8
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float keep = h2 ? u1[8 + i] : u1[i], send = h2 ? u1[i] : u1[8 + i];
    u2[i] = keep + __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(
                                                  __builtin_bit_cast(int, send), 0x401F));  // ^16
  }
  {
    const int src = (lane ^ 32) << 2;
    float r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float keep = h3 ? u2[4 + i] : u2[i], send = h3 ? u2[i] : u2[4 + i];
      r[i] = keep + __builtin_bit_cast(
                        float, __builtin_amdgcn_ds_bpermute(src, __builtin_bit_cast(int, send)));
    }
    // lane (q, h1 h2 h3) now holds columns 16 h1 + 8 h2 + 4 h3 + 0..3 of quad q
    red[wave][lane] = f32x4{r[0], r[1], r[2], r[3]};
  }
  if (t == 0) s_gave_up = 0;
  __syncthreads();

  // cross-wave sum and scale: this slice's partial of columns ct = t + NT c
  float mine[CPT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int ct = t + NT * c, qq = ct >> 5, cc = ct & 31;
    const int src = qq + 8 * (((cc >> 4) & 1) | (((cc >> 3) & 1) << 1) | (((cc >> 2) & 1) << 2));
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) {
      const f32x4 r = red[w][src];
      const int i = cc & 3;
      v += i == 0 ? r.x : i == 1 ? r.y : i == 2 ? r.z : r.w;
    }
    v *= scale_from_raw<ST>(sraw[c]);
    mine[c] = ev ? (v != v ? __builtin_nanf("") : v) : __builtin_nanf("");  // canonical NaN
  }
  uint64_t* strip_part = part + (int64_t)(j * S + strip) * P * SK_COLS;
  if (slice != P - 1) {  // a producer: hand the partial over, tagged, and leave
#pragma unroll
    for (int c = 0; c < CPT; ++c)
      if (ncol[c] >= 0)
        __hip_atomic_store(strip_part + (int64_t)slice * SK_COLS + (ncol[c] & 255),
                           (uint64_t)__builtin_bit_cast(u32, mine[c]) | ((uint64_t)tag << 32),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    return;
  }

  // the reducer: thread t reads columns 4 (t % 64) .. +3 of the slices
  // s = t / 64 (mod NWAVE) -- two 16-byte (value, tag) pairs each -- up to 8 * NWAVE
  // slices per round trip, until every pair carries the call's tag; the slice classes
  // are then added in class order in LDS
  __shared__ f32x4 red2[NWAVE][64];
  {
    constexpr int MAXB = 8;
    const rsrc_t pr = rsrc(strip_part, (u32)P * SK_COLS * 8u);
    const int cg = lane, so = wave;
    const bool cv = strip * SK_COLS + 4 * cg < N;  // whole column quads (N % 32 == 0)
    const u32x4 zero4 = {0u, 0u, 0u, 0u};
    f32x4 a4 = {0.f, 0.f, 0.f, 0.f};
    bool gave_up = false;
    for (int s0 = 0; s0 < P - 1 && !gave_up; s0 += NWAVE * MAXB) {
      u32x4 pa[MAXB], pb[MAXB];  // columns (4 cg, 4 cg + 1) and (4 cg + 2, 4 cg + 3)
      for (int poll = 0;; ++poll) {
        bool pending = false;
#pragma unroll
        for (int i = 0; i < MAXB; ++i) {  // past the last producer: re-read it, unused
          const u32 o = (u32)(min(s0 + so + NWAVE * i, P - 2) * SK_COLS + 4 * cg) * 8u;
          pa[i] = ld16_coherent(pr, o);
          pb[i] = ld16_coherent(pr, o + 16u);
        }
#pragma unroll
        for (int i = 0; i < MAXB; ++i)  // only the slices this thread owns
          pending |= cv && s0 + so + NWAVE * i < P - 1 &&
                     (pa[i].y != tag || pa[i].w != tag || pb[i].y != tag || pb[i].w != tag);
        if (!pending) break;
        if (poll >= max_polls) {
          gave_up = true;
          break;
        }
        // another pass issues the loads again: part is not __restrict__, so the
        // clobber below may have written it and the loads cannot be hoisted
        __builtin_amdgcn_s_sleep(1);
        asm volatile("" ::: "memory");
      }
      if (gave_up) break;
#pragma unroll
      for (int i = 0; i < MAXB; ++i) {
        const int sl = s0 + so + NWAVE * i;
        if (sl < P - 1 && cv) {
          // value words through scalars: a bit cast applied to an ext-vector component
          // directly reads component 0
          const u32 va[4] = {pa[i].x, pa[i].y, pa[i].z, pa[i].w};
          const u32 vb[4] = {pb[i].x, pb[i].y, pb[i].z, pb[i].w};
          a4 += f32x4{__builtin_bit_cast(float, va[0]), __builtin_bit_cast(float, va[2]),
                      __builtin_bit_cast(float, vb[0]), __builtin_bit_cast(float, vb[2])};
          const u32 o = (u32)(sl * SK_COLS + 4 * cg) * 8u;  // tags cleared for a replay
          __builtin_amdgcn_raw_buffer_store_b128(zero4, pr, o, 0, 0);
          __builtin_amdgcn_raw_buffer_store_b128(zero4, pr, o + 16u, 0, 0);
        }
      }
    }
    if (gave_up) {  // every tag of the strip cleared, including partials not seen yet
      for (int sl = so; sl < P - 1; sl += NWAVE) {
        const u32 o = (u32)(sl * SK_COLS + 4 * cg) * 8u;
        __builtin_amdgcn_raw_buffer_store_b128(zero4, pr, o, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b128(zero4, pr, o + 16u, 0, 0);
      }
      s_gave_up = 1;
    }
    red2[so][cg] = a4;
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    if (ncol[c] < 0) continue;
    const int n = ncol[c], nl = n & 255;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) {
      const f32x4 r = red2[w][nl >> 2];
      const int i = nl & 3;
      v += i == 0 ? r.x : i == 1 ? r.y : i == 2 ? r.z : r.w;
    }
    v += mine[c];  // the last slice's own partial
    if (s_gave_up) {
      v = __builtin_nanf("");
      if (t == 0 && c == 0) __hip_atomic_store(status, I4_ERR_HANDOFF, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
    }
    const int64_t o = (int64_t)j * N + n;
    if (ot == I4_F32) {
      if (bias) v += ((const float*)bias)[n];
      store_out<I4_F32>(out, o, v);
    } else if (ot == I4_F16) {
      if (bias) v += Half<I4_F16>::to_f32(((const uint16_t*)bias)[n]);
      store_out<I4_F16>(out, o, v);
    } else {
      if (bias) v += Half<I4_BF16>::to_f32(((const uint16_t*)bias)[n]);
      store_out<I4_BF16>(out, o, v);
    }
  }
}

// ---------------------------------------------------------------------------
// logical nibble / dequantised value of W[e][n][k] for both layouts
struct WView {
  const int32_t* packed;
  const void* scale;
  const int32_t* zeros;
  int64_t pes, ses, zes;
  int layout, group, st, E, N, K;
};

__device__ inline int awq_slot_of_col(int c8) {  // inverse of {0,2,4,6,1,3,5,7}
  return (c8 >> 1) + ((c8 & 1) << 2);
}

__device__ inline void nib_and_zero(const WView& w, int e, int n, int k, int& q, int& z,
                                    float& s) {
  const int NG = (w.K + w.group - 1) / w.group;
  const int g = k / w.group;
  if (w.layout == I4_LAYOUT_TILE) {
    const int SC = w.K >> 7, NZW = (NG + 7) >> 3, b = n >> 4, r = n & 15, c = k >> 5;
    const u32 word = (u32)w.packed[e * w.pes + (((int64_t)b * SC + (c >> 2)) * 16 + r) * 16 +
                                   ((k >> 3) & 3) * 4 + (c & 3)];
    q = (word >> (4 * awq_slot_of_col(k & 7))) & 15;  // interleaved nibbles
    z = w.zeros ? ((u32)w.zeros[e * w.zes + ((int64_t)b * NZW + (g >> 3)) * 16 + r] >>
                   (4 * (g & 7))) & 15
                : 8;
    const int64_t si = e * w.ses + ((int64_t)b * NG + g) * 16 + r;
    s = w.st == I4_F32 ? load_scale<I4_F32>(w.scale, si)
      : w.st == I4_F16 ? load_scale<I4_F16>(w.scale, si)
                       : load_scale<I4_BF16>(w.scale, si);
  } else if (w.layout == I4_LAYOUT_CT) {
    const u32 word = (u32)w.packed[e * w.pes + (int64_t)n * (w.K >> 3) + (k >> 3)];
    q = (word >> (4 * (k & 7))) & 15;
    if (w.zeros) {
      const int NZW = (NG + 7) >> 3;
      z = ((u32)w.zeros[e * w.zes + (int64_t)n * NZW + (g >> 3)] >> (4 * (g & 7))) & 15;
    } else {
      z = 8;
    }
    const int64_t si = e * w.ses + (int64_t)n * NG + g;
    s = w.st == I4_F32 ? load_scale<I4_F32>(w.scale, si)
      : w.st == I4_F16 ? load_scale<I4_F16>(w.scale, si)
                       : load_scale<I4_BF16>(w.scale, si);
  } else {
    const int NW = w.N >> 3, sl = awq_slot_of_col(n & 7);
    const u32 word = (u32)w.packed[e * w.pes + (int64_t)k * NW + (n >> 3)];
    q = (word >> (4 * sl)) & 15;
    if (w.zeros) {
      z = ((u32)w.zeros[e * w.zes + (int64_t)g * NW + (n >> 3)] >> (4 * sl)) & 15;
    } else {
      z = 8;
    }
    const int64_t si = e * w.ses + (int64_t)g * w.N + n;
    s = w.st == I4_F32 ? load_scale<I4_F32>(w.scale, si)
      : w.st == I4_F16 ? load_scale<I4_F16>(w.scale, si)
                       : load_scale<I4_BF16>(w.scale, si);
  }
}

// one thread per 8 consecutive k of one (e, n) row
__global__ __launch_bounds__(WG) void k_unpack(WView w, uint8_t* __restrict__ out, int ot_dequant,
                                               void* __restrict__ dq) {
  const int64_t i = (int64_t)blockIdx.x * WG + threadIdx.x;
  const int KW = w.K >> 3;
  const int64_t total = (int64_t)w.E * w.N * KW;
  if (i >= total) return;
  const int m = (int)(i % KW);
  const int64_t en = i / KW;
  const int n = (int)(en % w.N), e = (int)(en / w.N);
  for (int b = 0; b < 8; ++b) {
    int q, z;
    float s;
    const int k = 8 * m + b;
    nib_and_zero(w, e, n, k, q, z, s);
    const int64_t o = en * w.K + k;
    if (out) out[o] = (uint8_t)q;
    if (dq) {
      const float v = (float)(q - z) * s;
      if (ot_dequant == I4_F32) store_out<I4_F32>(dq, o, v);
      else if (ot_dequant == I4_F16) store_out<I4_F16>(dq, o, v);
      else store_out<I4_BF16>(dq, o, v);
    }
  }
}

// AWQ -> CT repack, one thread per CT word of expert e row n (packed part) and
// per (e, n, group) for scales / zeros.
__global__ __launch_bounds__(WG) void k_repack_awq(WView w, int32_t* __restrict__ dp,
                                                   void* __restrict__ ds, int32_t* __restrict__ dz,
                                                   int dst_rows, int row_off) {
  const int64_t i = (int64_t)blockIdx.x * WG + threadIdx.x;
  const int KW = w.K >> 3;
  const int NG = (w.K + w.group - 1) / w.group, NZW = (NG + 7) >> 3;
  const int64_t tot_w = (int64_t)w.E * w.N * KW;
  const int64_t tot_s = (int64_t)w.E * w.N * NG;
  const int64_t tot_z = (int64_t)w.E * w.N * NZW;
  if (i < tot_w) {
    const int m = (int)(i % KW);
    const int64_t en = i / KW;
    const int n = (int)(en % w.N), e = (int)(en / w.N);
    u32 word = 0;
    for (int b = 0; b < 8; ++b) {
      int q, z;
      float s;
      nib_and_zero(w, e, n, 8 * m + b, q, z, s);
      word |= (u32)q << (4 * b);
    }
    dp[((int64_t)e * dst_rows + row_off + n) * KW + m] = (int32_t)word;
  } else if (i < tot_w + tot_s) {
    const int64_t r = i - tot_w;
    const int g = (int)(r % NG);
    const int64_t en = r / NG;
    const int n = (int)(en % w.N), e = (int)(en / w.N);
    const int64_t src = e * w.ses + (int64_t)g * w.N + n;
    const int64_t dst = ((int64_t)e * dst_rows + row_off + n) * NG + g;
    if (w.st == I4_F32) ((float*)ds)[dst] = ((const float*)w.scale)[src];
    else ((uint16_t*)ds)[dst] = ((const uint16_t*)w.scale)[src];
  } else if (i < tot_w + tot_s + tot_z) {
    const int64_t r = i - tot_w - tot_s;
    const int zw = (int)(r % NZW);
    const int64_t en = r / NZW;
    const int n = (int)(en % w.N), e = (int)(en / w.N);
    u32 word = 0;
    for (int b = 0; b < 8; ++b) {
      const int g = 8 * zw + b;
      if (g >= NG) break;
      int q, z;
      float s;
      nib_and_zero(w, e, n, g * w.group, q, z, s);
      word |= (u32)z << (4 * b);
    }
    dz[((int64_t)e * dst_rows + row_off + n) * NZW + zw] = (int32_t)word;
  }
}

// CT or AWQ -> TILE, one thread per destination-ordered source item: the
// word m of (e, n) with its nibbles interleaved, then the scales and the zero
// words of (e, n).
__global__ __launch_bounds__(WG) void k_repack_tile(WView w, int32_t* __restrict__ dp,
                                                    void* __restrict__ ds,
                                                    int32_t* __restrict__ dz, int dst_rows,
                                                    int row_off) {
  const int64_t i = (int64_t)blockIdx.x * WG + threadIdx.x;
  const int KW = w.K >> 3, SC = w.K >> 7;
  const int NG = (w.K + w.group - 1) / w.group, NZW = (NG + 7) >> 3;
  const int DB = dst_rows >> 4;  // destination row blocks per expert
  const int64_t tot_w = (int64_t)w.E * w.N * KW;
  const int64_t tot_s = (int64_t)w.E * w.N * NG;
  const int64_t tot_z = dz ? (int64_t)w.E * w.N * NZW : 0;
  if (i < tot_w) {
    const int m = (int)(i % KW);
    const int64_t en = i / KW;
    const int n = (int)(en % w.N), e = (int)(en / w.N);
    u32 word = 0;  // column 8m + b in the AWQ nibble slot of b (interleaved)
    for (int b = 0; b < 8; ++b) {
      int q, z;
      float s;
      nib_and_zero(w, e, n, 8 * m + b, q, z, s);
      word |= (u32)q << (4 * awq_slot_of_col(b));
    }
    const int dn = row_off + n, c = m >> 2, j = m & 3;
    dp[((((int64_t)e * DB + (dn >> 4)) * SC + (c >> 2)) * 16 + (dn & 15)) * 16 + j * 4 + (c & 3)] =
        (int32_t)word;
  } else if (i < tot_w + tot_s) {
    const int64_t r = i - tot_w;
    const int g = (int)(r % NG);
    const int64_t en = r / NG;
    const int n = (int)(en % w.N), e = (int)(en / w.N);
    const int64_t src = w.layout == I4_LAYOUT_AWQ ? e * w.ses + (int64_t)g * w.N + n
                                                  : e * w.ses + (int64_t)n * NG + g;
    const int dn = row_off + n;
    const int64_t dst = (((int64_t)e * DB + (dn >> 4)) * NG + g) * 16 + (dn & 15);
    if (w.st == I4_F32) ((float*)ds)[dst] = ((const float*)w.scale)[src];
    else ((uint16_t*)ds)[dst] = ((const uint16_t*)w.scale)[src];
  } else if (i < tot_w + tot_s + tot_z) {
    const int64_t r = i - tot_w - tot_s;
    const int zw = (int)(r % NZW);
    const int64_t en = r / NZW;
    const int n = (int)(en % w.N), e = (int)(en / w.N);
    u32 word = 0;
    for (int b = 0; b < 8; ++b) {
      const int g = 8 * zw + b;
      if (g >= NG) break;
      int q, z;
      float s;
      nib_and_zero(w, e, n, g * w.group, q, z, s);
      word |= (u32)z << (4 * b);
    }
    const int dn = row_off + n;
    dz[(((int64_t)e * DB + (dn >> 4)) * NZW + zw) * 16 + (dn & 15)] = (int32_t)word;
  }
}

}  // namespace i4

// ===========================================================================
// host side
using namespace i4;

namespace {

inline bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }
inline bool half_dt(int d) { return d == I4_F16 || d == I4_BF16; }
inline bool any_dt(int d) { return d == I4_F32 || d == I4_F16 || d == I4_BF16; }


inline int64_t scale_ng(const i4_qweight* w) { return (w->K + w->group - 1) / w->group; }

inline int64_t dense_pes(const i4_qweight* w) { return (int64_t)w->N * w->K / 8; }
inline int64_t dense_ses(const i4_qweight* w) { return (int64_t)w->N * scale_ng(w); }
inline int64_t dense_zes(const i4_qweight* w) {  // CT and TILE hold the same words
  return w->layout == I4_LAYOUT_AWQ ? scale_ng(w) * (w->N / 8)
                                    : (int64_t)w->N * ((scale_ng(w) + 7) / 8);
}


}  // namespace

// validate an i4_qweight; fills dense strides when they are 0
int i4_check_weight(const i4_qweight* w, i4_qweight* norm) {
  if (!w || !w->packed || !w->scale) return I4_ERR_NULL;
  if (w->layout != I4_LAYOUT_CT && w->layout != I4_LAYOUT_AWQ && w->layout != I4_LAYOUT_TILE)
    return I4_ERR_LAYOUT;
  if (!any_dt(w->scale_dtype)) return I4_ERR_DTYPE;
  if (w->E < 1 || w->N < 1 || w->K < 32) return I4_ERR_SHAPE;
  if (w->K % 32 != 0 || w->K > 16384) return I4_ERR_SHAPE;
  if (w->layout == I4_LAYOUT_AWQ && w->N % 8 != 0) return I4_ERR_SHAPE;
  if (w->layout == I4_LAYOUT_TILE && (w->N % 16 != 0 || w->K % 128 != 0)) return I4_ERR_SHAPE;
  // a group spanning the whole row is one scale per output row (the per-channel
  // branch of quant/dequant.py:75-76); kernels index groups by powers of two
  int group = w->group;
  if (group >= w->K) {
    group = 32;
    while (group < w->K) group <<= 1;
  }
  if (group < 32 || (group & (group - 1)) != 0) return I4_ERR_GROUP;
  if (!al16(w->packed)) return I4_ERR_ALIGN;
  *norm = *w;
  norm->group = group;
  if (!norm->packed_estride) norm->packed_estride = dense_pes(w);
  if (!norm->scale_estride) norm->scale_estride = dense_ses(w);
  if (!norm->zeros_estride) norm->zeros_estride = dense_zes(w);
  if (w->E > 1 && (norm->packed_estride < dense_pes(w) || norm->scale_estride < dense_ses(w) ||
                   (w->zeros && norm->zeros_estride < dense_zes(w))))
    return I4_ERR_STRIDE;
  if (norm->packed_estride % 4 != 0) return I4_ERR_ALIGN;
  return I4_OK;
}

// CT GEMV launcher shared by i4_dq_gemv and i4_linear
template <int XT, int ST>
static int launch_gemv_ct_t(const void* x, int64_t x_stride, const i4_qweight* w,
                            const int32_t* sel, int k_sel, void* out, int ot, const void* bias,
                            hipStream_t s, const void* nw = nullptr, float eps = 0.f) {
  const int C = w->K / 32;
  const int L = gemv_lanes_per_row(C, w->N);
  const int rpw = WG / L;
  dim3 grid((w->N + rpw - 1) / rpw, k_sel);
  const size_t lds = (size_t)w->K * 2 + (size_t)C * 8;
  const int gshift = i4_group_shift(w->group);
#define I4_GEMV_CASE(L_, NORM_)                                                                 \
  if (L == L_) {                                                                                \
    hipLaunchKernelGGL((k_gemv_ct<XT, ST, L_, NORM_>), grid, dim3(WG), lds, s,                  \
                       (const uint16_t*)x, x_stride, w->packed, w->packed_estride, w->scale,    \
                       w->scale_estride, w->zeros, w->zeros_estride, sel, w->E, w->N, w->K,     \
                       gshift, out, ot, bias, (const uint16_t*)nw, eps);                        \
    return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;                             \
  }
  if (nw) {  // K <= 4096: C <= 128 lanes' worth, L in 8..32
    I4_GEMV_CASE(8, true) I4_GEMV_CASE(16, true) I4_GEMV_CASE(32, true)
    return I4_ERR_SHAPE;
  }
  I4_GEMV_CASE(4, false) I4_GEMV_CASE(8, false) I4_GEMV_CASE(16, false) I4_GEMV_CASE(32, false)
  I4_GEMV_CASE(64, false)
#undef I4_GEMV_CASE
  return I4_ERR_SHAPE;
}

int i4_launch_gemv_ct(const void* x, int xt, int64_t x_stride, const i4_qweight* w,
                      const int32_t* sel, int k_sel, void* out, int ot, const void* bias,
                      hipStream_t s) {
#define I4_GEMV_DT(XT_, ST_)                                                             \
  if (xt == XT_ && w->scale_dtype == ST_)                                                \
    return launch_gemv_ct_t<XT_, ST_>(x, x_stride, w, sel, k_sel, out, ot, bias, s);
  I4_GEMV_DT(I4_F16, I4_F32) I4_GEMV_DT(I4_F16, I4_F16) I4_GEMV_DT(I4_F16, I4_BF16)
  I4_GEMV_DT(I4_BF16, I4_F32) I4_GEMV_DT(I4_BF16, I4_F16) I4_GEMV_DT(I4_BF16, I4_BF16)
#undef I4_GEMV_DT
  return I4_ERR_DTYPE;
}

// the AWQ GEMV reads scales 16 bytes at a time
inline bool awq_scales_aligned(const i4_qweight& w) {
  const int sb = w.scale_dtype == I4_F32 ? 4 : 2;
  return ((uintptr_t)w.scale & 15) == 0 && (w.E == 1 || (w.scale_estride * sb) % 16 == 0);
}

// rows per block of the AWQ GEMV: one block per thread up to K = 256 RB, RB | group
inline int awq_rows_per_block(int K, int group) {
  int rb = 2;
  while (rb < 16 && rb * WG < K) rb *= 2;
  return rb < group ? rb : group;
}

template <int XT, int ST>
static int launch_gemv_awq_t(const void* x, int64_t x_stride, const i4_qweight* w,
                             const int32_t* sel, int k_sel, void* out, int ot, const void* bias,
                             hipStream_t s) {
  const int RB = awq_rows_per_block(w->K, w->group);
  int gshift = 0;
  while ((1 << gshift) < w->group) ++gshift;
  const dim3 grid(w->N / 8, k_sel);
#define I4_AWQ_CASE(RB_)                                                                        \
  if (RB == RB_) {                                                                              \
    hipLaunchKernelGGL((k_gemv_awq<XT, ST, RB_>), grid, dim3(WG), 0, s, (const uint16_t*)x,     \
                       x_stride, w->packed, w->packed_estride, w->scale, w->scale_estride,      \
                       w->zeros, w->zeros_estride, sel, w->E, w->N, w->K, gshift, out, ot, bias); \
    return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;                             \
  }
  I4_AWQ_CASE(2) I4_AWQ_CASE(4) I4_AWQ_CASE(8) I4_AWQ_CASE(16)
#undef I4_AWQ_CASE
  return I4_ERR_SHAPE;
}

// Split-K plan of the AWQ GEMV: waves per workgroup, row pairs per thread
// (slice = 16 * waves * pairs rows), strips, slices; waves == 0: the shape
// keeps the K-complete kernel.  Measured on one MI355X with the hand-over inside an
// XCD (each GEMV one of 64 distinct weight copies, back to back in a graph): the split
// launch takes 5.75 us at 2048 -> 4096 and 6.3 us at 4096 -> 2048 (through memory
// across XCDs: 7.2 / 8.1; K-complete: 8.5-9.6), but 6.0 us at 2048 -> 768 and 5.5 at
// 2048 -> 512 with at least 64 workgroups against 5.8 / 4.9 K-complete.  So the split
// is taken only where the K-complete launch fills more than 2048 rows of lines per CU
// (K rows per workgroup, N / 8 workgroups per row of x over 256 CUs), and only for up
// to kSplitRows rows of x (decode: the plan was measured at one row) whose partials
// fit kSplitBytes; more rows run K-complete.  Its slice is
// the largest of 128 / 64 / 32 rows that divides K and the group: a slice's loads
// are one round trip at any of these sizes, and fewer slices make fewer partials to
// hand over.
static constexpr int kSplitRows = 8;
static constexpr size_t kSplitBytes = (size_t)8 << 20;
struct AwqSplit {
  int nwave, ppt, S, P;
};
// workspace of a split-K plan: the header (status word), then the (value, tag)
// partials [row][strip][slice][256] of 8 bytes
static size_t awq_split_bytes(const AwqSplit& p, int k_sel) {
  if (!p.nwave) return 0;
  return SK_HEAD + (size_t)k_sel * p.S * p.P * SK_COLS * sizeof(uint64_t);
}
static AwqSplit awq_split_plan(const i4_qweight& w, int k_sel) {
  AwqSplit p{0, 0, 0, 0};
  if (w.layout != I4_LAYOUT_AWQ || w.N % 32 != 0 || k_sel < 1 || k_sel > kSplitRows) return p;
  if (w.zeros && (((uintptr_t)w.zeros & 15) || (w.E > 1 && w.zeros_estride % 4))) return p;
  const int64_t rounds = ((int64_t)(w.N / 8) * k_sel + 255) / 256;
  if ((int64_t)w.K * rounds <= 2048) return p;
  const int S = (w.N / 8 + 31) / 32;
  static const int opts[3][2] = {{4, 2}, {4, 1}, {2, 1}};
  for (const auto& o : opts) {
    const int ks = 16 * o[0] * o[1];
    if (w.K % ks != 0 || w.group % ks != 0) continue;
    p = AwqSplit{o[0], o[1], S, w.K / ks};
    break;
  }
  if (awq_split_bytes(p, k_sel) > kSplitBytes) p = AwqSplit{0, 0, 0, 0};
  return p;
}

// the tag of one call of the split-K GEMV: a process-wide count, never 0
static std::atomic<uint32_t> g_call_tag{0};
static u32 next_call_tag() {
  u32 t = ++g_call_tag;
  while (t == 0) t = ++g_call_tag;
  return t;
}

template <int XT, int ST>
static int launch_gemv_awq_sk_t(const void* x, int64_t x_stride, const i4_qweight* w,
                                const int32_t* sel, int k_sel, void* out, int ot,
                                const void* bias, const AwqSplit& p, void* ws, int max_polls,
                                bool reducers_only, hipStream_t s) {
  int gshift = 0;
  while ((1 << gshift) < w->group) ++gshift;
  const dim3 grid(reducers_only ? p.S : 8 * ((p.S + 7) / 8) * p.P, k_sel);
  int32_t* status = (int32_t*)ws;
  uint64_t* part = (uint64_t*)((char*)ws + SK_HEAD);
  const u32 tag = next_call_tag();
#define I4_SK_CASE(NW_, PPT_)                                                                     \
  if (p.nwave == NW_ && p.ppt == PPT_) {                                                          \
    hipLaunchKernelGGL((k_gemv_awq_sk<XT, ST, NW_, PPT_>), grid, dim3(64 * NW_), 0, s,            \
                       (const uint16_t*)x, x_stride, w->packed, w->packed_estride, w->scale,      \
                       w->scale_estride, w->zeros, w->zeros_estride, sel, w->E, w->N, gshift,     \
                       p.S, p.P, part, out, ot, bias, max_polls, tag, status,                     \
                       (int)reducers_only);                                                       \
    return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;                               \
  }
  I4_SK_CASE(4, 2) I4_SK_CASE(4, 1) I4_SK_CASE(2, 1)
#undef I4_SK_CASE
  return I4_ERR_SHAPE;
}

// AWQ GEMV: split along K when the caller passes the plan's workspace, else
// the K-complete kernel (no workspace)
static int launch_gemv_awq(const void* x, int xt, int64_t x_stride, const i4_qweight* w,
                           const int32_t* sel, int k_sel, void* out, int ot, const void* bias,
                           void* ws, size_t ws_bytes, hipStream_t s, int max_polls = kAwqPolls,
                           bool reducers_only = false) {
  const AwqSplit p = awq_split_plan(*w, k_sel);
  if (p.nwave && ws) {
    if (ws_bytes < awq_split_bytes(p, k_sel)) return I4_ERR_WORKSPACE;
    if ((uintptr_t)ws & 255) return I4_ERR_ALIGN;
#define I4_AWQ_DT(XT_, ST_)                                                                   \
  if (xt == XT_ && w->scale_dtype == ST_)                                                     \
    return launch_gemv_awq_sk_t<XT_, ST_>(x, x_stride, w, sel, k_sel, out, ot, bias, p, ws,   \
                                          max_polls, reducers_only, s);
    I4_AWQ_DT(I4_F16, I4_F32) I4_AWQ_DT(I4_F16, I4_F16) I4_AWQ_DT(I4_F16, I4_BF16)
    I4_AWQ_DT(I4_BF16, I4_F32) I4_AWQ_DT(I4_BF16, I4_F16) I4_AWQ_DT(I4_BF16, I4_BF16)
#undef I4_AWQ_DT
    return I4_ERR_DTYPE;
  }
  if (reducers_only) return I4_ERR_WORKSPACE;  // only a split launch has reducers
#define I4_AWQ_DT(XT_, ST_)                                                              \
  if (xt == XT_ && w->scale_dtype == ST_)                                                \
    return launch_gemv_awq_t<XT_, ST_>(x, x_stride, w, sel, k_sel, out, ot, bias, s);
  I4_AWQ_DT(I4_F16, I4_F32) I4_AWQ_DT(I4_F16, I4_F16) I4_AWQ_DT(I4_F16, I4_BF16)
  I4_AWQ_DT(I4_BF16, I4_F32) I4_AWQ_DT(I4_BF16, I4_F16) I4_AWQ_DT(I4_BF16, I4_BF16)
#undef I4_AWQ_DT
  return I4_ERR_DTYPE;
}

extern "C" {

size_t i4_dq_gemv_workspace_bytes(const i4_qweight* w, int k_sel) {
  i4_qweight nw;
  if (!w || i4_check_weight(w, &nw) != I4_OK) return 0;
  return awq_split_bytes(awq_split_plan(nw, k_sel), k_sel);
}

int i4_dq_gemv(const void* x, int x_dtype, int64_t x_stride, const i4_qweight* w,
               const int32_t* sel, int k_sel, void* out, int out_dtype, void* workspace,
               size_t workspace_bytes, hipStream_t stream) {
  return i4_dq_gemv_bounded(x, x_dtype, x_stride, w, sel, k_sel, out, out_dtype, workspace,
                            workspace_bytes, kAwqPolls, 0, stream);
}

int i4_dq_gemv_bounded(const void* x, int x_dtype, int64_t x_stride, const i4_qweight* w,
                       const int32_t* sel, int k_sel, void* out, int out_dtype, void* workspace,
                       size_t workspace_bytes, int max_polls, int reducers_only,
                       hipStream_t stream) {
  if (max_polls < 0) return I4_ERR_SHAPE;
  i4_qweight nw;
  int rc = i4_check_weight(w, &nw);
  if (rc) return rc;
  if (!x || !sel || !out) return I4_ERR_NULL;
  if (!half_dt(x_dtype) || !any_dt(out_dtype)) return I4_ERR_DTYPE;
  if (k_sel < 1 || k_sel > 65535 || x_stride < 0) return I4_ERR_SHAPE;
  if (x_stride != 0 && x_stride < nw.K) return I4_ERR_STRIDE;
  if (!al16(x) || (x_stride * 2) % 16 != 0) return I4_ERR_ALIGN;
  if (nw.layout == I4_LAYOUT_TILE) return I4_ERR_LAYOUT;  // the MoE kernels' layout
  if (nw.layout == I4_LAYOUT_AWQ && !awq_scales_aligned(nw)) return I4_ERR_ALIGN;
  if (nw.layout == I4_LAYOUT_CT) {
    if (reducers_only) return I4_ERR_LAYOUT;  // only the AWQ split launch hands over
    return i4_launch_gemv_ct(x, x_dtype, x_stride, &nw, sel, k_sel, out, out_dtype, nullptr,
                             stream);
  }
  return launch_gemv_awq(x, x_dtype, x_stride, &nw, sel, k_sel, out, out_dtype, nullptr,
                         workspace, workspace_bytes, stream, max_polls, reducers_only != 0);
}

int i4_rmsnorm_linear(const void* x, int x_dtype, int M, const void* norm_w, float eps,
                      const i4_qweight* w, const void* bias, void* y, int y_dtype,
                      hipStream_t stream) {
  i4_qweight nw;
  int rc = i4_check_weight(w, &nw);
  if (rc) return rc;
  if (!x || !y || !norm_w) return I4_ERR_NULL;
  if (!half_dt(x_dtype) || !any_dt(y_dtype)) return I4_ERR_DTYPE;
  if (nw.layout != I4_LAYOUT_CT) return I4_ERR_LAYOUT;
  if (M < 1 || M > 65535 || nw.K > 4096 || nw.K % 8) return I4_ERR_SHAPE;
  if (!al16(x) || !al16(norm_w)) return I4_ERR_ALIGN;
  nw.E = 1;
#define I4_NL_DT(XT_, ST_)                                                                   \
  if (x_dtype == XT_ && nw.scale_dtype == ST_)                                               \
    return launch_gemv_ct_t<XT_, ST_>(x, nw.K, &nw, nullptr, M, y, y_dtype, bias, stream,     \
                                      norm_w, eps);
  I4_NL_DT(I4_F16, I4_F32) I4_NL_DT(I4_F16, I4_F16) I4_NL_DT(I4_F16, I4_BF16)
  I4_NL_DT(I4_BF16, I4_F32) I4_NL_DT(I4_BF16, I4_F16) I4_NL_DT(I4_BF16, I4_BF16)
#undef I4_NL_DT
  return I4_ERR_DTYPE;
}

size_t i4_linear_workspace_bytes(const i4_qweight* w, int M) {
  if (w && w->layout == I4_LAYOUT_TILE && M >= 1) return linear_tile_workspace_bytes(M, w->N, w->K);
  return i4_dq_gemv_workspace_bytes(w, M);
}

int i4_linear(const void* x, int x_dtype, int M, const i4_qweight* w, const void* bias, void* y,
              int y_dtype, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  i4_qweight nw;
  int rc = i4_check_weight(w, &nw);
  if (rc) return rc;
  if (!x || !y) return I4_ERR_NULL;
  if (!half_dt(x_dtype) || !any_dt(y_dtype)) return I4_ERR_DTYPE;
  if (M < 1 || M > 65535) return I4_ERR_SHAPE;
  if (!al16(x)) return I4_ERR_ALIGN;
  if (nw.layout == I4_LAYOUT_TILE) {  // several rows: MFMA over 64-row tiles
    if (nw.E != 1) return I4_ERR_SHAPE;
    TW tw{nw.packed, nw.scale, nw.zeros, nw.packed_estride, nw.scale_estride,
          nw.zeros_estride, i4_group_shift(nw.group), 1, nw.N, nw.K};
#define I4_LIN_DT(XT_, ST_)                                                                 \
  if (x_dtype == XT_ && nw.scale_dtype == ST_)                                              \
    return launch_mfma_linear<XT_, ST_>(x, M, tw, bias, y, y_dtype, workspace, workspace_bytes, \
                                        stream);
    I4_LIN_DT(I4_F16, I4_F32) I4_LIN_DT(I4_F16, I4_F16) I4_LIN_DT(I4_F16, I4_BF16)
    I4_LIN_DT(I4_BF16, I4_F32) I4_LIN_DT(I4_BF16, I4_F16) I4_LIN_DT(I4_BF16, I4_BF16)
#undef I4_LIN_DT
    return I4_ERR_DTYPE;
  }
  nw.E = 1;
  if (nw.layout == I4_LAYOUT_CT)
    return i4_launch_gemv_ct(x, x_dtype, nw.K, &nw, nullptr, M, y, y_dtype, bias, stream);
  if (!awq_scales_aligned(nw)) return I4_ERR_ALIGN;
  return launch_gemv_awq(x, x_dtype, nw.K, &nw, nullptr, M, y, y_dtype, bias, workspace,
                         workspace_bytes, stream);
}

static WView make_view(const i4_qweight& w) {
  WView v;
  v.packed = w.packed;
  v.scale = w.scale;
  v.zeros = w.zeros;
  v.pes = w.packed_estride;
  v.ses = w.scale_estride;
  v.zes = w.zeros_estride;
  v.layout = w.layout;
  v.group = w.group;
  v.st = w.scale_dtype;
  v.E = w.E;
  v.N = w.N;
  v.K = w.K;
  return v;
}

int i4_unpack(const i4_qweight* w, uint8_t* out, hipStream_t stream) {
  i4_qweight nw;
  int rc = i4_check_weight(w, &nw);
  if (rc) return rc;
  if (!out) return I4_ERR_NULL;
  const int64_t total = (int64_t)nw.E * nw.N * (nw.K / 8);
  hipLaunchKernelGGL(k_unpack, dim3((unsigned)((total + WG - 1) / WG)), dim3(WG), 0, stream,
                     make_view(nw), out, 0, (void*)nullptr);
  return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;
}

int i4_dequant(const i4_qweight* w, void* out, int out_dtype, hipStream_t stream) {
  i4_qweight nw;
  int rc = i4_check_weight(w, &nw);
  if (rc) return rc;
  if (!out) return I4_ERR_NULL;
  if (!any_dt(out_dtype)) return I4_ERR_DTYPE;
  const int64_t total = (int64_t)nw.E * nw.N * (nw.K / 8);
  hipLaunchKernelGGL(k_unpack, dim3((unsigned)((total + WG - 1) / WG)), dim3(WG), 0, stream,
                     make_view(nw), (uint8_t*)nullptr, out_dtype, out);
  return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;
}

int i4_repack_awq_to_ct(const i4_qweight* src, int32_t* dst_packed, void* dst_scale,
                        int32_t* dst_zeros, int dst_rows, int row_offset, hipStream_t stream) {
  i4_qweight nw;
  int rc = i4_check_weight(src, &nw);
  if (rc) return rc;
  if (nw.layout != I4_LAYOUT_AWQ) return I4_ERR_LAYOUT;
  if (!dst_packed || !dst_scale || !dst_zeros) return I4_ERR_NULL;
  if (row_offset < 0 || dst_rows < row_offset + nw.N) return I4_ERR_SHAPE;
  const int NG = (nw.K + nw.group - 1) / nw.group;
  const int64_t total = (int64_t)nw.E * nw.N * (nw.K / 8 + NG + (NG + 7) / 8);
  hipLaunchKernelGGL(k_repack_awq, dim3((unsigned)((total + WG - 1) / WG)), dim3(WG), 0, stream,
                     make_view(nw), dst_packed, dst_scale, dst_zeros, dst_rows, row_offset);
  return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;
}

int i4_repack_tile(const i4_qweight* src, int32_t* dst_packed, void* dst_scale,
                   int32_t* dst_zeros, int dst_rows, int row_offset, hipStream_t stream) {
  i4_qweight nw;
  int rc = i4_check_weight(src, &nw);
  if (rc) return rc;
  if (nw.layout == I4_LAYOUT_TILE) return I4_ERR_LAYOUT;
  if (!dst_packed || !dst_scale || (nw.zeros && !dst_zeros)) return I4_ERR_NULL;
  if (nw.K % 128 != 0 || dst_rows % 16 != 0 || row_offset % 16 != 0) return I4_ERR_SHAPE;
  if (row_offset < 0 || dst_rows < row_offset + nw.N) return I4_ERR_SHAPE;
  if (!al16(dst_packed)) return I4_ERR_ALIGN;
  const int NG = (nw.K + nw.group - 1) / nw.group;
  const int64_t total =
      (int64_t)nw.E * nw.N * (nw.K / 8 + NG + (dst_zeros ? (NG + 7) / 8 : 0));
  hipLaunchKernelGGL(k_repack_tile, dim3((unsigned)((total + WG - 1) / WG)), dim3(WG), 0, stream,
                     make_view(nw), dst_packed, dst_scale, dst_zeros, dst_rows, row_offset);
  return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;
}

}  // extern "C"
