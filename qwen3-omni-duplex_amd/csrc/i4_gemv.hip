// int4 dequant-GEMV kernels for gfx950 and their C-ABI entry points.
//
//   k_gemv_ct      gathered GEMV on the compressed-tensors layout
//                  (replaces _dq_gemv_kernel, triton_dequant_gemv.py:32-82)
//   k_gemv_awq     split-K GEMV straight on AutoAWQ packing + k_reduce_split
//   k_unpack       raw nibbles in logical [E][N][K] order (unpack4,
//                  fused_packed_moe.py:54-65)
//   k_dequant      dense (q - z) * s (FusedPackedMoE._dequant, :183-189)
//   k_repack_awq   AWQ -> CT(+zeros) conversion done once at load time
//
// CT GEMV work split: L lanes cooperate on one output row, lane l of the row
// owns the 32-column chunks c = l, l + L, l + 2L, ... and streams each chunk
// with one 16-byte load, so the L lanes of a row read L*16 contiguous bytes
// (L >= 8 keeps every load a whole 128-byte line).  A 256-thread workgroup
// therefore owns 256/L consecutive rows of one selected expert; grid.y is the
// selected-expert slot.  All weight loads of a round are issued before the
// activation row is staged, so the staging latency hides under the stream.
#include "i4_common.h"
#include "i4_launch.h"
#include "i4_moe_launch.h"

namespace i4 {

static constexpr int WG = 256;
static constexpr int ROUND = 4;  // chunks per lane whose loads are in flight together

// NORM: each workgroup first applies the RMSNorm with weight nw to its staged x
// row (K <= 4096), with the arithmetic of k_rmsnorm_t (same thread -> word map
// and reduction order), so the result equals i4_rmsnorm followed by the GEMV.
template <int XT, int ST, int L, bool NORM>
__global__ __launch_bounds__(WG) void k_gemv_ct(
    const uint16_t* __restrict__ x, int64_t x_stride, const int32_t* __restrict__ packed,
    int64_t p_es, const void* __restrict__ scale, int64_t s_es,
    const int32_t* __restrict__ zeros, int64_t z_es, const int32_t* __restrict__ sel, int E,
    int N, int K, int gshift, void* __restrict__ out, int ot, const void* __restrict__ bias,
    const uint16_t* __restrict__ nw, float eps) {
  extern __shared__ __align__(16) unsigned char lds[];
  constexpr int RPW = WG / L;
  const int C = K >> 5, KW = K >> 3;
  const int NG = (C + (1 << gshift) - 1) >> gshift, NZW = (NG + 7) >> 3;
  const int cpl = (C + L - 1) / L;
  u32x4* xs = (u32x4*)lds;
  float2* sums = (float2*)(lds + (size_t)K * 2);

  const int j = blockIdx.y;
  const int rl = threadIdx.x / L, cl = threadIdx.x % L;
  const int n = blockIdx.x * RPW + rl;
  const bool rv = n < N;
  const int e = sel ? sel[j] : 0;
  if ((unsigned)e >= (unsigned)E) {  // bad expert id: never dereference it
    if (rv && cl == 0) {
      if (ot == I4_F32) store_out<I4_F32>(out, (int64_t)j * N + n, __builtin_nanf(""));
      else if (ot == I4_F16) store_out<I4_F16>(out, (int64_t)j * N + n, __builtin_nanf(""));
      else store_out<I4_BF16>(out, (int64_t)j * N + n, __builtin_nanf(""));
    }
    return;
  }
  const int nn = rv ? n : 0;
  RowPtr rp;
  rp.p = packed + e * p_es + (int64_t)nn * KW;
  rp.s = scale_at<ST>(scale, e * s_es + (int64_t)nn * NG);
  rp.z = zeros ? (const u32*)zeros + e * z_es + (int64_t)nn * NZW : kSymZeros;
  const uint16_t* xrow = x + (int64_t)j * x_stride;
  const u32 mg = magic_v<XT>();
  Stager<XT> st(1, K);  // activation loads first, weight loads behind them
  auto row_of = [&](int) { return xrow; };
  st.issue(row_of, 0);
  u32x4 gv[2];
  if constexpr (NORM) {
#pragma unroll
    for (int u = 0; u < 2; ++u) gv[u] = ldg16(nw + 8 * min(u * WG + (int)threadIdx.x, st.total - 1));
  }

  float row = 0.f;
  for (int r0 = 0; r0 < cpl; r0 += ROUND) {
    Chunk ch[ROUND];
#pragma unroll
    for (int i = 0; i < ROUND; ++i) ch[i] = load_chunk<ST>(rp, min(cl + (r0 + i) * L, C - 1), gshift);
    if (r0 == 0) {
      if constexpr (NORM) {
        __shared__ float s_ss[WG / 64];
        float ss = 0.f;
#pragma unroll
        for (int u = 0; u < 2; ++u)
          if (u * WG + (int)threadIdx.x < st.total) ss += sumsq8<XT>(st.d[u]);
        ss = group_sum<64>(ss);
        if ((threadIdx.x & 63) == 0) s_ss[threadIdx.x >> 6] = ss;
        __syncthreads();
        const float r =
            1.0f / sqrtf(((s_ss[0] + s_ss[1]) + (s_ss[2] + s_ss[3])) / (float)K + eps);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          st.d[u].x = norm_pair<XT>(st.d[u].x, gv[u].x, r);
          st.d[u].y = norm_pair<XT>(st.d[u].y, gv[u].y, r);
          st.d[u].z = norm_pair<XT>(st.d[u].z, gv[u].z, r);
          st.d[u].w = norm_pair<XT>(st.d[u].w, gv[u].w, r);
        }
      }
      st.commit(0, xs, sums);
      st.rest(row_of, xs, sums);
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < ROUND; ++i) {
      const int c = cl + (r0 + i) * L;
      if (c < C)
        row += chunk_dot<XT, ST>(ch[i], xs[c], xs[C + c], xs[2 * C + c], xs[3 * C + c], sums[c], c,
                                 gshift, mg);
    }
  }
  row = group_sum<L>(row);
  if (rv && cl == 0) {
    const int64_t o = (int64_t)j * N + n;
    if (ot == I4_F32) {
      if (bias) row += ((const float*)bias)[n];
      store_out<I4_F32>(out, o, row);
    } else if (ot == I4_F16) {
      if (bias) row += Half<I4_F16>::to_f32(((const uint16_t*)bias)[n]);
      store_out<I4_F16>(out, o, row);
    } else {
      if (bias) row += Half<I4_BF16>::to_f32(((const uint16_t*)bias)[n]);
      store_out<I4_BF16>(out, o, row);
    }
  }
}

// ---------------------------------------------------------------------------
// AWQ split-K GEMV.  Thread t of a workgroup owns column word cw = tile*32 +
// (t & 31) (8 output columns) and k-slot t >> 5; the workgroup covers rows
// [k0, k0 + KS) of the weight.  A k-slot processes row pairs (k, k+1); the
// two words are merged byte-wise with v_perm_b32 so that every column gets a
// (row k, row k+1) pair for v_dot2.  Partial sums go to part[split][j][N].
static constexpr int AWQ_TILE = 32;  // column words per workgroup
static constexpr int AWQ_SLOTS = WG / AWQ_TILE;
__constant__ int kAwqOrder[8] = {0, 2, 4, 6, 1, 3, 5, 7};

template <int XT>
__global__ __launch_bounds__(WG) void k_gemv_awq(
    const uint16_t* __restrict__ x, int64_t x_stride, const int32_t* __restrict__ qw, int64_t q_es,
    const void* __restrict__ scales, int64_t s_es, int st, const int32_t* __restrict__ qz,
    int64_t z_es, const int32_t* __restrict__ sel, int E, int N, int K, int group, int KS,
    float* __restrict__ part) {
  __shared__ u32 xs2[2048];          // (x[k], x[k+1]) pairs of this split, KS <= 4096
  __shared__ float red[AWQ_SLOTS][AWQ_TILE][8];
  const int NW = N >> 3;
  const int j = blockIdx.z, split = blockIdx.y, nsplit = gridDim.y;
  const int t = threadIdx.x, lc = t & (AWQ_TILE - 1), slot = t / AWQ_TILE;
  const int cw = blockIdx.x * AWQ_TILE + lc;
  const bool cv = cw < NW;
  const int k0 = split * KS;
  const int kend = min(K, k0 + KS);
  const int e = sel ? sel[j] : 0;
  const bool ev = (unsigned)e < (unsigned)E;
  float* dst = part + ((int64_t)split * gridDim.z + j) * N;
  if (!ev) {
    if (cv && slot == 0)
      for (int i = 0; i < 8; ++i) dst[8 * cw + i] = __builtin_nanf("");
    return;
  }
  // stage x pairs of this split
  const uint16_t* xrow = x + (int64_t)j * x_stride;
  for (int p = t; p < (kend - k0) / 2; p += WG) xs2[p] = *(const u32*)(xrow + k0 + 2 * p);
  __syncthreads();

  const int32_t* qe = qw + e * q_es;
  const int32_t* ze = qz ? qz + e * z_es : nullptr;
  const int64_t se = e * s_es;
  float acc_tot[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc_tot[i] = 0.f;
  constexpr u32 MK = 0x000F000Fu;
  const u32 mg = magic_v<XT>();
  const u32 ONE2 = XT == I4_F16 ? 0x3C003C00u : 0x3F803F80u;  // (1.0, 1.0)
  // One quantisation group at a time, its rows in batches of RB row pairs per
  // k-slot (128 rows): every weight word, the zero word and the 8 scales of a
  // batch are loaded before any is used (indices clamped, so the loads are
  // unconditional), then consumed -- one memory round trip per batch.
  constexpr int RB = 8;
  const int cwc = cv ? cw : NW - 1;
  for (int gk = k0; gk < kend; gk += group) {
    const int g = gk / group;
    const int gend = min(kend, gk + group);
    const u32 zw = ze ? (u32)ze[(int64_t)g * NW + cwc] : 0x88888888u;
    float sv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t si = se + (int64_t)g * N + 8 * cwc + kAwqOrder[i];
      sv[i] = st == I4_F32 ? load_scale<I4_F32>(scales, si)
            : st == I4_F16 ? load_scale<I4_F16>(scales, si)
                           : load_scale<I4_BF16>(scales, si);
    }
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.f;
    float S = 0.f;
    for (int kb0 = gk + 2 * slot; kb0 < gend; kb0 += 2 * AWQ_SLOTS * RB) {
      u32 w0[RB], w1[RB];
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const int k = min(kb0 + 2 * AWQ_SLOTS * r, gend - 2);
        w0[r] = (u32)qe[(int64_t)k * NW + cwc];
        w1[r] = (u32)qe[(int64_t)(k + 1) * NW + cwc];
      }
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const int k = kb0 + 2 * AWQ_SLOTS * r;
        if (k < gend) {
          const u32 xp = xs2[(k - k0) >> 1];
          S = Half<XT>::dot2(xp, ONE2, S);
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            // byte b of w0 -> bits 0..7, byte b of w1 -> bits 16..23
            const u32 sel_b = 0x0C000C00u | (u32)(b) | ((u32)(4 + b) << 16);
            const u32 tb = __builtin_amdgcn_perm(w1[r], w0[r], sel_b);
            acc[2 * b] = Half<XT>::dot2((tb & MK) | mg, xp, acc[2 * b]);
            acc[2 * b + 1] = Half<XT>::dot2(((tb >> 4) & MK) | mg, xp, acc[2 * b + 1]);
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float z = (float)((zw >> (4 * i)) & 15u);
      acc_tot[i] += sv[i] * (acc[i] - (Half<XT>::MAGIC + z) * S);
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) red[slot][lc][i] = acc_tot[i];
  __syncthreads();
  {
    const int ol = t >> 3, oi = t & 7;  // 32 words x 8 slots = 256 outputs
    const int ocw = blockIdx.x * AWQ_TILE + ol;
    if (ocw < NW) {
      float s = 0.f;
      for (int sl = 0; sl < AWQ_SLOTS; ++sl) s += red[sl][ol][oi];
      dst[8 * ocw + kAwqOrder[oi]] = s;
    }
  }
  (void)nsplit;
}

// out[j][n] = sum_s part[s][j][n] (+ bias[n]), fixed split order
__global__ __launch_bounds__(WG) void k_reduce_split(const float* __restrict__ part, int nsplit,
                                                     int64_t total, int N, void* __restrict__ out,
                                                     int ot, const void* __restrict__ bias) {
  const int64_t i = (int64_t)blockIdx.x * WG + threadIdx.x;
  if (i >= total) return;
  float s = 0.f;
  for (int p = 0; p < nsplit; ++p) s += part[(int64_t)p * total + i];
  const int n = (int)(i % N);
  if (ot == I4_F32) {
    if (bias) s += ((const float*)bias)[n];
    store_out<I4_F32>(out, i, s);
  } else if (ot == I4_F16) {
    if (bias) s += Half<I4_F16>::to_f32(((const uint16_t*)bias)[n]);
    store_out<I4_F16>(out, i, s);
  } else {
    if (bias) s += Half<I4_BF16>::to_f32(((const uint16_t*)bias)[n]);
    store_out<I4_BF16>(out, i, s);
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

inline int lanes_per_row(int C) {
  int L = 4;
  while (L * 2 <= C && L < 64) L *= 2;
  while (L > 8 && C < 3 * L) L /= 2;
  return L;
}

inline int64_t scale_ng(const i4_qweight* w) { return (w->K + w->group - 1) / w->group; }

inline int64_t dense_pes(const i4_qweight* w) { return (int64_t)w->N * w->K / 8; }
inline int64_t dense_ses(const i4_qweight* w) { return (int64_t)w->N * scale_ng(w); }
inline int64_t dense_zes(const i4_qweight* w) {  // CT and TILE hold the same words
  return w->layout == I4_LAYOUT_AWQ ? scale_ng(w) * (w->N / 8)
                                    : (int64_t)w->N * ((scale_ng(w) + 7) / 8);
}

inline int awq_split_rows(const i4_qweight* w) {
  int gps = 1;
  while ((int64_t)w->K > (int64_t)w->group * gps * 32) gps *= 2;
  int ks = w->group * gps;
  if (ks > 4096) ks = 4096 / w->group * w->group;
  return ks;
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
  if (w->group < 32 || (w->group & (w->group - 1)) != 0) return I4_ERR_GROUP;
  if (!al16(w->packed)) return I4_ERR_ALIGN;
  *norm = *w;
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
  const int L = lanes_per_row(C);
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

static int launch_gemv_awq(const void* x, int xt, int64_t x_stride, const i4_qweight* w,
                           const int32_t* sel, int k_sel, void* out, int ot, const void* bias,
                           void* ws, size_t ws_bytes, hipStream_t s) {
  const int KS = awq_split_rows(w);
  const int nsplit = (w->K + KS - 1) / KS;
  const size_t need = (size_t)nsplit * k_sel * w->N * sizeof(float);
  if (!ws || ws_bytes < need) return I4_ERR_WORKSPACE;
  dim3 grid((w->N / 8 + AWQ_TILE - 1) / AWQ_TILE, nsplit, k_sel);
  if (xt == I4_F16)
    hipLaunchKernelGGL((k_gemv_awq<I4_F16>), grid, dim3(WG), 0, s, (const uint16_t*)x, x_stride,
                       w->packed, w->packed_estride, w->scale, w->scale_estride, w->scale_dtype,
                       w->zeros, w->zeros_estride, sel, w->E, w->N, w->K, w->group, KS,
                       (float*)ws);
  else
    hipLaunchKernelGGL((k_gemv_awq<I4_BF16>), grid, dim3(WG), 0, s, (const uint16_t*)x, x_stride,
                       w->packed, w->packed_estride, w->scale, w->scale_estride, w->scale_dtype,
                       w->zeros, w->zeros_estride, sel, w->E, w->N, w->K, w->group, KS,
                       (float*)ws);
  if (hipGetLastError() != hipSuccess) return I4_ERR_LAUNCH;
  const int64_t total = (int64_t)k_sel * w->N;
  hipLaunchKernelGGL(k_reduce_split, dim3((unsigned)((total + WG - 1) / WG)), dim3(WG), 0, s,
                     (const float*)ws, nsplit, total, w->N, out, ot, bias);
  return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;
}

extern "C" {

size_t i4_dq_gemv_workspace_bytes(const i4_qweight* w, int k_sel) {
  if (!w || w->layout != I4_LAYOUT_AWQ || k_sel < 1 || w->group < 32) return 0;
  const int KS = awq_split_rows(w);
  const int nsplit = (w->K + KS - 1) / KS;
  return (size_t)nsplit * k_sel * w->N * sizeof(float);
}

int i4_dq_gemv(const void* x, int x_dtype, int64_t x_stride, const i4_qweight* w,
               const int32_t* sel, int k_sel, void* out, int out_dtype, void* workspace,
               size_t workspace_bytes, hipStream_t stream) {
  i4_qweight nw;
  int rc = i4_check_weight(w, &nw);
  if (rc) return rc;
  if (!x || !sel || !out) return I4_ERR_NULL;
  if (!half_dt(x_dtype) || !any_dt(out_dtype)) return I4_ERR_DTYPE;
  if (k_sel < 1 || k_sel > 65535 || x_stride < 0) return I4_ERR_SHAPE;
  if (x_stride != 0 && x_stride < nw.K) return I4_ERR_STRIDE;
  if (!al16(x) || (x_stride * 2) % 16 != 0) return I4_ERR_ALIGN;
  if (nw.layout == I4_LAYOUT_TILE) return I4_ERR_LAYOUT;  // the MoE kernels' layout
  if (nw.layout == I4_LAYOUT_CT)
    return i4_launch_gemv_ct(x, x_dtype, x_stride, &nw, sel, k_sel, out, out_dtype, nullptr,
                             stream);
  return launch_gemv_awq(x, x_dtype, x_stride, &nw, sel, k_sel, out, out_dtype, nullptr,
                         workspace, workspace_bytes, stream);
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
