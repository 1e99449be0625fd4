// Grouped (T > 1) expert projections on MFMA, I4_LAYOUT_TILE weights.
//
// The tokens of one expert form the M dimension (m-blocks of 16), weight rows
// the N dimension (n-blocks of 16 = one tile row block), and K is walked in
// 128-column superchunks.  v_mfma_f32_16x16x32_{f16,bf16}: lane (r, j) =
// (l % 16, l / 16) supplies A[m = r][8 columns] and B[8 columns][n = r] and
// receives D[4 j + i][r], i < 4.  MFMA step t of superchunk s contracts chunk
// 4s + t: B is word j of that chunk (component t of the lane's 16-byte tile
// word) decoded to 8 halves in the (c, c+4) pair order, A the same 8 columns
// of the token (k = 128 s + 32 t + 8 j) permuted to match.
//   fp16: B holds q - z exactly ((M + q) - (M + z), one packed half add per
//         pair) and a group ends with res += s D.
//   bf16: B holds M + q exactly (gfx950 has no packed bf16 add) and a group
//         ends with res += s D - s (M + z) S_m, S_m the sum of token m's
//         activations over the group.
// Every product is exact and accumulation is fp32, as in the decode kernels.
//
// k_tile_mfma_s (entries of <= 16 tokens, one m-block): every lane loads its
// own A words straight from global memory (the four waves of a workgroup hit
// the same L1 lines), no LDS and no barrier; the weights and activations of
// the next two superchunks are in flight while one is multiplied (three-slot
// register ring, unrolled so every slot index is static, loads issued
// unconditionally so that the waits before each use stay partial).
// k_tile_mfma (entries of <= 64 tokens): the activation tile of a superchunk
// is staged once per workgroup in LDS (double buffered, token stride 272 B so
// the 16 tokens of an MFMA fall on distinct banks), weights in the same
// three-slot ring.
//   GATEUP: NB/2 blocks of gate rows and the same up rows per wave, SiLU in
//           the epilogue, act[pos] in the activation dtype; 32 NB row pairs
//           per workgroup.
//   DOWN:   NB blocks of output rows per wave, ys[slot] in fp32; 64 NB rows
//           per workgroup.
#include "i4_moe_launch.h"

namespace i4 {

static constexpr int MF_TSTRIDE = 17;  // uint4 per staged token row (16 + 1 pad)

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

template <int XT> __device__ inline f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (XT == I4_F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// 8 exact halves M + q of one CT word, in the (c, c+4) pair order
template <int XT> __device__ inline u32x4 decode8(u32 w) {
  constexpr u32 MK = 0x000F000Fu, MG = Half<XT>::MAGIC2;
  return u32x4{(w & MK) | MG, ((w >> 4) & MK) | MG, ((w >> 8) & MK) | MG, ((w >> 12) & MK) | MG};
}

// fp16 pair (M + q0, M + q1) + nz, nz = (-(M + z), -(M + z)): exactly (q0 - z, q1 - z)
__device__ inline u32 sub_zero(u32 p, u32 nz) {
  return __builtin_bit_cast(u32, __builtin_bit_cast(f16x2, p) + __builtin_bit_cast(f16x2, nz));
}

// B operand of step t for one n-block
template <int XT> __device__ inline u32x4 b_operand(u32 word, u32 zw, int g) {
  u32x4 b = decode8<XT>(word);
  if constexpr (XT == I4_F16) {
    const u32 nz = (0xE400u | ((zw >> (4 * (g & 7))) & 15u)) * 0x00010001u;
    b.x = sub_zero(b.x, nz);
    b.y = sub_zero(b.y, nz);
    b.z = sub_zero(b.z, nz);
    b.w = sub_zero(b.w, nz);
  }
  return b;
}

// first row block of n-block nb of wave `wave` in column tile `tile`
template <bool GATEUP, int NB>
__device__ inline int nblock(int tile, int wave, int nb, int I) {
  if constexpr (GATEUP)
    return tile * (2 * NB) + (NB / 2) * wave + (nb % (NB / 2)) + (nb >= NB / 2 ? (I >> 4) : 0);
  else
    return tile * (4 * NB) + NB * wave + nb;
}

template <int XT, int ST, bool GB, int NB> struct MSlot {
  TSlot<GB> w[NB];
  u32x4 a[4];
};

// group correction of one n-block's accumulator (rows m = 4 j + i of column r)
template <int XT, int ST>
__device__ inline void correct(f32x4& res, const f32x4& d, u32 sraw, u32 zw, int g,
                               const float (&sm)[4]) {
  const float sv = scale_from_raw<ST>(sraw);
  if constexpr (XT == I4_F16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) res[i] = fmaf(sv, d[i], res[i]);
  } else {
    const float bv = -sv * (Half<XT>::MAGIC + (float)((zw >> (4 * (g & 7))) & 15u));
#pragma unroll
    for (int i = 0; i < 4; ++i) res[i] = fmaf(sv, d[i], fmaf(bv, sm[i], res[i]));
  }
}

template <int XT, int ST, bool GB, bool GATEUP, int NB>
__global__ __launch_bounds__(256) void k_tile_mfma_s(
    const uint16_t* __restrict__ src, int topk, const int4* __restrict__ entries,
    const int* __restrict__ n_entries, const int32_t* __restrict__ perm, TW w, int I,
    uint16_t* __restrict__ act, float* __restrict__ ys) {
  constexpr bool EXACT = XT == I4_F16;
  constexpr int COLS = GATEUP ? 32 * NB : 64 * NB;
  static_assert(!GATEUP || NB % 2 == 0, "gate_up pairs gate and up blocks");
  if ((int)blockIdx.y >= *n_entries) return;
  const int4 en = entries[blockIdx.y];
  const int e = en.x, pos0 = en.y, cnt = en.z;
  const int K = w.K, SC = K >> 7;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, ln = lane & 15, kb = lane >> 4;
  const bool ev = (unsigned)e < (unsigned)w.E;
  const int ee = ev ? e : 0;
  TileRow tr[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
    tr[nb] = tile_row<ST>(w, ee, nblock<GATEUP, NB>(blockIdx.x, wave, nb, I), ln, kb);
  // A row of this lane: token ln of the entry (clamped; rows >= cnt are not stored)
  const uint16_t* xrow;
  if constexpr (GATEUP) xrow = src + (int64_t)(perm[pos0 + min(ln, cnt - 1)] / topk) * K;
  else xrow = src + (int64_t)(pos0 + min(ln, cnt - 1)) * K;
  xrow += 8 * kb;

  using Slot = MSlot<XT, ST, GB, NB>;
  auto issue = [&](int sc, Slot& sl) {
    sc = min(sc, SC - 1);  // past the end: the last superchunk again, an L2 hit
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) sl.w[nb] = tile_load<ST, GB>(tr[nb], sc, w.gshift);
#pragma unroll
    for (int t = 0; t < 4; ++t) sl.a[t] = ldg16(xrow + 128 * sc + 32 * t);
  };
  f32x4 res[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) res[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  // bf16: S of rows m = 4 j + i from this lane's partial sums p (token ln)
  auto rows_sum = [&](float p, float (&sm)[4]) {
    const float tot = kgroup_sum(p);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      sm[i] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((4 * kb + i) << 2,
                                                                     __builtin_bit_cast(int, tot)));
  };
  auto compute = [&](int sc, const Slot& sl) {
    f32x4 d[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) d[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
    float pg = 0.f;  // bf16, GB: partial activation sum over the superchunk
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int g = (4 * sc + t) >> w.gshift;
      const u32x4 a = pair_order(sl.a[t]);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        d[nb] = mfma16<XT>(a, b_operand<XT>(word_t(sl.w[nb].w, t), sl.w[nb].z, g), d[nb]);
      if constexpr (!GB) {
        float sm[4] = {0.f, 0.f, 0.f, 0.f};
        if constexpr (!EXACT) rows_sum(sum8<XT>(sl.a[t]).y, sm);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          correct<XT, ST>(res[nb], d[nb], sl.w[nb].s[t], sl.w[nb].z, g, sm);
          d[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      } else if constexpr (!EXACT) {
        pg += sum8<XT>(sl.a[t]).y;
      }
    }
    if constexpr (GB) {
      const int g = (4 * sc) >> w.gshift;
      float sm[4] = {0.f, 0.f, 0.f, 0.f};
      if constexpr (!EXACT) rows_sum(pg, sm);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) correct<XT, ST>(res[nb], d[nb], sl.w[nb].s[0], sl.w[nb].z, g, sm);
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

template <int XT, int ST, bool GB, bool GATEUP, int NB>
__global__ __launch_bounds__(256) void k_tile_mfma(
    const uint16_t* __restrict__ src, int topk, const int4* __restrict__ entries,
    const int* __restrict__ n_entries, const int32_t* __restrict__ perm, TW w, int I,
    uint16_t* __restrict__ act, float* __restrict__ ys) {
  constexpr bool EXACT = XT == I4_F16;
  constexpr int COLS = GATEUP ? 32 * NB : 64 * NB;
  static_assert(!GATEUP || NB % 2 == 0, "gate_up pairs gate and up blocks");
  __shared__ u32x4 xs[2][MF_TOK * MF_TSTRIDE];
  __shared__ float xsum[2][MF_TOK * 4];  // bf16: per token and chunk
  if ((int)blockIdx.y >= *n_entries) return;
  const int4 en = entries[blockIdx.y];
  const int e = en.x, pos0 = en.y, cnt = en.z;
  const int K = w.K, SC = K >> 7;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, ln = lane & 15, kb = lane >> 4;
  const bool ev = (unsigned)e < (unsigned)w.E;
  const int ee = ev ? e : 0;
  const int nmb = (cnt + 15) >> 4;
  TileRow tr[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
    tr[nb] = tile_row<ST>(w, ee, nblock<GATEUP, NB>(blockIdx.x, wave, nb, I), ln, kb);
  // staging role: token tk, chunk kc (words 4 kc .. 4 kc + 3) of the superchunk
  const int tk = threadIdx.x >> 2, kc = threadIdx.x & 3;
  const uint16_t* xrow;
  if constexpr (GATEUP) xrow = src + (int64_t)(perm[pos0 + min(tk, cnt - 1)] / topk) * K;
  else xrow = src + (int64_t)(pos0 + min(tk, cnt - 1)) * K;
  xrow += 32 * kc;
  u32x4 xd[4];
  auto issue_x = [&](int sc) {
    sc = min(sc, SC - 1);
#pragma unroll
    for (int q = 0; q < 4; ++q) xd[q] = ldg16(xrow + 128 * sc + 8 * q);
  };
  auto commit_x = [&](int buf) {
    float sm = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      xs[buf][tk * MF_TSTRIDE + 4 * kc + q] = pair_order(xd[q]);
      if constexpr (!EXACT) sm += sum8<XT>(xd[q]).y;
    }
    if constexpr (!EXACT) xsum[buf][4 * tk + kc] = sm;
  };
  using WSlot = TSlot<GB>[NB];
  auto issue_w = [&](int sc, WSlot& sl) {
    sc = min(sc, SC - 1);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) sl[nb] = tile_load<ST, GB>(tr[nb], sc, w.gshift);
  };
  f32x4 res[4][NB];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) res[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  // S of rows 16 mb + 4 j + i over chunks [t0, t0 + nt) of the staged superchunk
  auto rows_sum = [&](int buf, int mb, int t0, int nt, float (&sm)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float* p = &xsum[buf][4 * (16 * mb + 4 * kb + i)];
      float v = 0.f;
      for (int t = t0; t < t0 + nt; ++t) v += p[t];
      sm[i] = v;
    }
  };
  auto compute = [&](int sc, const WSlot& sl, int buf) {
    f32x4 d[4][NB];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) d[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int g = (4 * sc + t) >> w.gshift;
      u32x4 b[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) b[nb] = b_operand<XT>(word_t(sl[nb].w, t), sl[nb].z, g);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        if (mb < nmb) {
          const u32x4 a = xs[buf][(16 * mb + ln) * MF_TSTRIDE + 4 * t + kb];
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) d[mb][nb] = mfma16<XT>(a, b[nb], d[mb][nb]);
        }
      }
      if constexpr (!GB) {
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
          if (mb < nmb) {
            float sm[4] = {0.f, 0.f, 0.f, 0.f};
            if constexpr (!EXACT) rows_sum(buf, mb, t, 1, sm);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
              correct<XT, ST>(res[mb][nb], d[mb][nb], sl[nb].s[t], sl[nb].z, g, sm);
              d[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
          }
        }
      }
    }
    if constexpr (GB) {
      const int g = (4 * sc) >> w.gshift;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        if (mb < nmb) {
          float sm[4] = {0.f, 0.f, 0.f, 0.f};
          if constexpr (!EXACT) rows_sum(buf, mb, 0, 4, sm);
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            correct<XT, ST>(res[mb][nb], d[mb][nb], sl[nb].s[0], sl[nb].z, g, sm);
        }
      }
    }
  };
  // one superchunk: stage its activations (loaded one step earlier), load the
  // next step's, multiply, refill this weight slot three superchunks ahead
  auto step = [&](int sc, WSlot& sl) {
    const int buf = sc & 1;
    if (sc < SC) {
      commit_x(buf);
      __syncthreads();
    }
    issue_x(sc + 1);  // unconditional (clamped), like every load of the ring
    if (sc < SC) compute(sc, sl, buf);
    issue_w(sc + 3, sl);
  };
  WSlot s0, s1, s2;
  issue_w(0, s0);
  issue_w(1, s1);
  issue_w(2, s2);
  issue_x(0);
  for (int sc = 0; sc < SC; sc += 3) {
    step(sc, s0);
    step(sc + 1, s1);
    step(sc + 2, s2);
  }
  // epilogue: lane holds rows m = 16 mb + 4 j + i of column r
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

// ---------------------------------------------------------------------------
template <int XT, int ST, bool GB, bool GATEUP>
static int mfma_t(bool small, int max_entries, const void* src, int topk, const int4* ent,
                  const int* nent, const int32_t* perm, const TW& w, int I, void* act, float* ys,
                  hipStream_t s) {
  const int cols = GATEUP ? 32 * MF_NB : 64 * MF_NB;
  const dim3 grid((GATEUP ? I : w.N) / cols, max_entries);
  if (small)
    hipLaunchKernelGGL((k_tile_mfma_s<XT, ST, GB, GATEUP, MF_NB>), grid, dim3(256), 0, s,
                       (const uint16_t*)src, topk, ent, nent, perm, w, I, (uint16_t*)act, ys);
  else
    hipLaunchKernelGGL((k_tile_mfma<XT, ST, GB, GATEUP, MF_NB>), grid, dim3(256), 0, s,
                       (const uint16_t*)src, topk, ent, nent, perm, w, I, (uint16_t*)act, ys);
  return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;
}

template <int XT, int ST>
int launch_mfma_gate_up(bool small, int max_entries, const void* x, int topk, const int4* ent,
                        const int* nent, const int32_t* perm, const TW& w, int I, void* act,
                        hipStream_t s) {
  if (w.gshift >= 2)
    return mfma_t<XT, ST, true, true>(small, max_entries, x, topk, ent, nent, perm, w, I, act,
                                      nullptr, s);
  return mfma_t<XT, ST, false, true>(small, max_entries, x, topk, ent, nent, perm, w, I, act,
                                     nullptr, s);
}

template <int XT, int ST>
int launch_mfma_down(bool small, int max_entries, const void* act, const int4* ent,
                     const int* nent, const int32_t* perm, const TW& w, float* ys, hipStream_t s) {
  if (w.gshift >= 2)
    return mfma_t<XT, ST, true, false>(small, max_entries, act, 0, ent, nent, perm, w, 0, nullptr,
                                       ys, s);
  return mfma_t<XT, ST, false, false>(small, max_entries, act, 0, ent, nent, perm, w, 0, nullptr,
                                      ys, s);
}

#define I4_INST(XT_, ST_)                                                                       \
  template int launch_mfma_gate_up<XT_, ST_>(bool, int, const void*, int, const int4*,          \
                                             const int*, const int32_t*, const TW&, int, void*, \
                                             hipStream_t);                                      \
  template int launch_mfma_down<XT_, ST_>(bool, int, const void*, const int4*, const int*,      \
                                          const int32_t*, const TW&, float*, hipStream_t);
I4_INST(I4_F16, I4_F32) I4_INST(I4_F16, I4_F16) I4_INST(I4_F16, I4_BF16)
I4_INST(I4_BF16, I4_F32) I4_INST(I4_BF16, I4_F16) I4_INST(I4_BF16, I4_BF16)
#undef I4_INST

}  // namespace i4
