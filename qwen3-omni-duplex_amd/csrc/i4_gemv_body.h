// Body of the CT dequant-GEMV (k_gemv_ct), shared by the GEMV launches and by
// launches that run it behind a producer of their activation row.
//
// L lanes cooperate on one output row; lane l of the row owns the 32-column
// chunks c = l, l + L, l + 2L, ... and streams each chunk with one 16-byte
// load, so the L lanes of a row read L*16 contiguous bytes (L >= 8 keeps every
// load a whole 128-byte line).  A 256-thread workgroup therefore owns 256/L
// consecutive rows of one selected expert.  All weight loads of a round are
// issued before the activation row is staged, so the staging latency hides
// under the stream.
#pragma once

#include "i4_common.h"
#include "i4_router_body.h"

namespace i4 {

static constexpr int GEMV_WG = 256;
static constexpr int GEMV_ROUND = 4;  // chunks per lane whose loads are in flight together

// NORM: each workgroup first applies the RMSNorm with weight nw to its staged x
// row (K <= 4096), with the arithmetic of k_rmsnorm_t (same thread -> word map
// and reduction order), so the result equals i4_rmsnorm followed by the GEMV.
// POLL: x (one row, K <= 8192) is written by earlier workgroups of the same
// launch and holds the pending pattern until then; the workgroup issues its
// first round of weight loads, then polls x (poll_rows) instead of loading it.
// Rows of a workgroup whose wait gives up come out NaN, and I4_ERR_HANDOFF goes to
// *status (nullable).
// HANDOFF: out (ot = XT) is read by later workgroups of the same launch: the
// workgroup's rows are gathered in LDS and written through to memory as whole
// 16-byte stores where they are aligned (else value by value), NaN in canonical form (so the pending
// pattern never appears in finished values).  Same arithmetic as the plain store.
// TAG (with HANDOFF): out is instead an array of (value pair, tag) words, 8 bytes per
// two rows, every pair of the workgroup's rows stored with `tag` (N a multiple of the
// workgroup's RPW rows): the readers wait for the tag of their call, so the buffer
// needs no pending pattern.
// COMP (with NORM, K = 2048): x is the residual row of a decode layer whose experts left
// one output row per slot (slot_y [8][K], routing weights slot_w [8]); the row is
// completed first, x + sum_k w[k] y[k] (slot_sum8: the single-launch combine's arithmetic,
// so equal to it bit for bit), its loads issued ahead of the weight stream, and workgroup
// bx = 0 writes the completed row to h_out.
template <int XT, int ST, int L, bool NORM, bool POLL, bool HANDOFF = false, bool TAG = false,
          bool COMP = false>
__device__ __forceinline__ void gemv_ct_body(
    int bx, int j, const uint16_t* __restrict__ x, int64_t x_stride,
    const int32_t* __restrict__ packed, int64_t p_es, const void* __restrict__ scale,
    int64_t s_es, const int32_t* __restrict__ zeros, int64_t z_es,
    const int32_t* __restrict__ sel, int E, int N, int K, int gshift, void* __restrict__ out,
    int ot, const void* __restrict__ bias, const uint16_t* __restrict__ nw, float eps,
    unsigned char* lds, int max_polls, int32_t* __restrict__ status = nullptr, u32 tag = 0,
    const uint16_t* __restrict__ slot_y = nullptr, const float* __restrict__ slot_w = nullptr,
    uint16_t* __restrict__ h_out = nullptr) {
  constexpr int WG = GEMV_WG, ROUND = GEMV_ROUND;
  static_assert(!COMP || (NORM && !POLL), "the completed row is normalised as it is staged");
  static_assert(!(NORM && POLL), "a polled row is used as it arrives");
  static_assert(!TAG || HANDOFF, "tags belong to a hand-over");
  constexpr int RPW = WG / L;
  const int C = K >> 5, KW = K >> 3;
  const int NG = (C + (1 << gshift) - 1) >> gshift, NZW = (NG + 7) >> 3;
  const int cpl = (C + L - 1) / L;
  u32x4* xs = (u32x4*)lds;
  float2* sums = (float2*)(lds + (size_t)K * 2);

  const int rl = threadIdx.x / L, cl = threadIdx.x % L;
  const int n = bx * RPW + rl;
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
  // COMP: thread t's word of the residual row and of the 8 slot rows (K = 2048: one word)
  u32x4 cres, cy[COMP ? 8 : 1];
  float cw[COMP ? 8 : 1];
  if constexpr (COMP) {
    const int idx = (int)threadIdx.x;
    cres = ldg16(xrow + 8 * idx);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      cy[k] = ldg16(slot_y + (int64_t)k * K + 8 * idx);
      cw[k] = slot_w[k];
    }
  } else if constexpr (!POLL) {
    st.issue(row_of, 0);
  }
  u32x4 gv[2];
  if constexpr (NORM) {
#pragma unroll
    for (int u = 0; u < 2; ++u) gv[u] = ldg16(nw + 8 * min(u * WG + (int)threadIdx.x, st.total - 1));
  }

  bool late = false;
  float row = 0.f;
  // A round takes R = ROUND chunks per lane, or 2 where at most 2 are left (a row of 2L
  // chunks issues no dead loads).  A FULL round has every chunk inside the row for every
  // lane: no per-lane test, so the round's dot is one basic block whose LDS reads all go
  // out before the first product.  The chunks add up in the same order in every form.
  // The activation row is staged once, after the first round's weight loads are issued.
  auto stage = [&]() {
    if constexpr (POLL) late = poll_rows<XT>(st, xrow, max_polls);
    if constexpr (COMP) {
      st.d[0] = slot_sum8<XT, 8>(cres, cy, cw);
      st.d[1] = st.d[0];  // K = 2048: one word per thread
      if (h_out && bx == 0) *(u32x4*)(h_out + 8 * (int)threadIdx.x) = st.d[0];
    }
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
    if constexpr (!POLL) st.rest(row_of, xs, sums);
    __syncthreads();
  };
  auto round = [&](int r0, auto rr, auto full) {
    constexpr int R = decltype(rr)::value;
    constexpr bool FULL = decltype(full)::value;
    Chunk ch[R];
#pragma unroll
    for (int i = 0; i < R; ++i)
      ch[i] = load_chunk<ST>(rp, FULL ? cl + (r0 + i) * L : min(cl + (r0 + i) * L, C - 1), gshift);
    if (r0 == 0) stage();
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int c = cl + (r0 + i) * L;
      if (FULL || c < C)
        row += chunk_dot<XT, ST>(ch[i], xs[c], xs[C + c], xs[2 * C + c], xs[3 * C + c], sums[c], c,
                                 gshift, mg);
    }
  };
  using R2 = std::integral_constant<int, 2>;
  using RF = std::integral_constant<int, ROUND>;
  for (int r0 = 0; r0 < cpl;) {
    // the shape of the round (wave-uniform)
    const bool two = cpl - r0 <= 2;
    const bool full = (r0 + (two ? 2 : ROUND)) * L <= C;
    if (two && full) round(r0, R2{}, std::true_type{});
    else if (two) round(r0, R2{}, std::false_type{});
    else if (full) round(r0, RF{}, std::true_type{});
    else round(r0, RF{}, std::false_type{});
    r0 += two ? 2 : ROUND;
  }
  row = group_sum<L>(row);
  if constexpr (POLL) {  // a wait that gave up is reported (status nullable)
    if (late && status && threadIdx.x == 0)
      __hip_atomic_store(status, I4_ERR_HANDOFF, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if constexpr (HANDOFF) {
    __shared__ __align__(16) uint16_t s_y[RPW];
    if (rv && cl == 0) {
      if (late) row = __builtin_nanf("");
      if (bias) row += Half<XT>::to_f32(((const uint16_t*)bias)[n]);
      const uint16_t b = Half<XT>::from_f32(row);
      s_y[rl] = row != row ? Half<XT>::QNAN : b;
    }
    __syncthreads();
    const int n0 = bx * RPW, nv = min(RPW, N - n0);
    if constexpr (TAG) {
      static_assert(RPW % 4 == 0, "whole 16-byte stores of two (pair, tag) words");
      // thread i: pairs 2i, 2i + 1 of the workgroup's rows as {pair, tag, pair, tag}
      if ((int)threadIdx.x < RPW / 4) {
        const u32* sp = (const u32*)s_y + 2 * threadIdx.x;
        const u32 p0 = sp[0], p1 = sp[1];
        const rsrc_t r = rsrc((u32*)out + ((int64_t)j * N + n0), (u32)RPW * 4u);
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{p0, tag, p1, tag}, r, (u32)threadIdx.x * 16u,
                                               0, kCoherent);
      }
      return;
    }
    uint16_t* dst = (uint16_t*)out + (int64_t)j * N + n0;
    if (RPW % 8 == 0 && nv == RPW && ((uintptr_t)dst & 15) == 0) {
      if ((int)threadIdx.x < RPW / 8) {
        const rsrc_t r = rsrc(dst, (u32)RPW * 2u);
        __builtin_amdgcn_raw_buffer_store_b128(((const u32x4*)s_y)[threadIdx.x], r,
                                               (u32)threadIdx.x * 16u, 0, kCoherent);
      }
    } else if ((int)threadIdx.x < nv) {
      st_coherent(dst + threadIdx.x, s_y[threadIdx.x]);
    }
    return;
  }
  if (rv && cl == 0) {
    if (late) row = __builtin_nanf("");
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

// lanes per output row of an N-row GEMV (4..64): 3+ chunks per lane when the row is
// long enough, 2+ (twice the lanes, twice the workgroups) for N <= 1024 and N > 4096.
// Measured at K = 2048 on one MI355X: 2048 -> 768 3.71 -> 3.53 us, 2048 -> 512 3.32 ->
// 3.17, the decode step's q|k|v with its input norm (N = 5120) 0.3 us faster per layer;
// q_proj 2048 -> 4096 slower (3.80 -> 4.17), so that band keeps 3+ chunks; and
// 4096-value rows stay at 32 lanes (64: o_proj 4096 -> 2048 3.88 -> 4.30 us).
inline int gemv_lanes_per_row(int C, int N) {
  const int per = N <= 1024 || N > 4096 ? 2 : 3;
  int L = 4;
  while (L * 2 <= C && L < 64) L *= 2;
  while (L > 8 && (C < per * L || (L > 32 && C < 3 * L))) L /= 2;
  return L;
}

}  // namespace i4
