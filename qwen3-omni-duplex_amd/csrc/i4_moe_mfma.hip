// Grouped (T > 1) expert projections on MFMA, I4_LAYOUT_TILE weights.
//
// The tokens of one expert form the M dimension (m-blocks of 16), weight rows
// the N dimension (n-blocks of 16 = one tile row block), and K is walked in
// 128-column superchunks.  v_mfma_f32_16x16x32_{f16,bf16}: lane (r, j) =
// (l % 16, l / 16) supplies A[m = r][8 columns] and B[8 columns][n = r] and
// receives D[4 j + i][r], i < 4.  MFMA step t of superchunk s contracts chunk
// 4s + t: B is word j of that chunk (component t of the lane's 16-byte tile
// word) decoded to 8 halves, A the same 8 columns of the token (k = 128 s +
// 32 t + 8 j) as they lie in memory: the tile word's interleaved nibbles put
// the decoded halves in column order.
//   fp16: B holds q - z exactly ((M + q) - (M + z), one packed half add per
//         pair) and a group ends with res += s D.  Large entries (four
//         m-blocks) instead fold the scale into B with one packed multiply,
//         so each dequantised weight is rounded once to fp16 (relative error
//         <= 2^-11, the numerics of dequantise-then-multiply) and the MFMA
//         accumulates straight into the result: no second accumulator, which
//         keeps a 64-token entry within 128 VGPRs.
//   bf16: B holds M + q exactly (gfx950 has no packed bf16 add or multiply)
//         and a group ends with res += s D - s (M + z) S_m, S_m the sum of
//         token m's activations over the group.
// Accumulation is fp32; apart from the fold every product is exact.
//
// All global reads are raw buffer loads: one descriptor per operand (an
// expert's weights, scales and zero words; the activation rows), per-lane
// offsets computed once, and the superchunk / group offsets in scalar
// registers, so the loop spends no vector instructions on addresses.  A
// weight without zero points reads its zero words through an empty
// descriptor (every load returns 0) and ORs in the symmetric 0x88888888.
//
// k_tile_mfma<..., NB, MB>: one entry (<= 16 MB tokens of one expert) times
// one column tile per workgroup.  The activation tile of a superchunk (16 MB
// tokens x 128 columns) is loaded once per workgroup and staged in LDS
// (double buffered, 256-byte token rows with the words XOR-swizzled by token so
// the 16 tokens of an MFMA fall on distinct banks); every wave streams its own
// NB n-blocks through a
// three-slot register ring (unrolled so every slot index is static, loads
// issued unconditionally so that the waits before each use stay partial).
// Small entries (<= 16 tokens) run MB = 1 with NB = 4 where the rows allow,
// so a wave keeps 12 KB of weights in flight; large entries (<= 64 tokens)
// run MB = 4, NB = 2, each decoded weight feeding up to four MFMAs.
//   GATEUP: NB/2 blocks of gate rows and the same up rows per wave, SiLU in
//           the epilogue, act[pos] in the activation dtype; 32 NB row pairs
//           per workgroup.
//   DOWN:   NB blocks of output rows per wave, ys[slot] rounded to the
//           activation dtype (the reference's y.to(x.dtype), fused_packed_moe.py:262); 64 NB rows
//           per workgroup.
#include "i4_moe_launch.h"

namespace i4 {

// Staged activations: token m's 16 words of a superchunk are one 256-byte row, word w
// at slot w ^ (m & 15) (xs_at).  An MFMA operand load (lanes = 16 tokens x 4
// words) and a staging store (16 lanes = 4 tokens x 4 words) each touch every bank
// once per 16 lanes; measured on gfx950, the swizzled rows read at 4.4 cycles per
// wave-wide 16-byte load against 8.1 with a one-word pad per row.
static constexpr int MF_TSTRIDE = 16;  // uint4 per staged token row
__device__ inline int xs_at(int m, int w) { return m * MF_TSTRIDE + (w ^ (m & 15)); }

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
__device__ inline u32x4 bload16(rsrc_t r, u32 voff, int soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
}
// the same past the L1 (sc1): sees what other CUs of the launch wrote through
__device__ inline u32x4 bload16_coherent(rsrc_t r, u32 voff, int soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kCoherent);
}
__device__ inline u32 bload4(rsrc_t r, u32 voff, int soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}
template <int ST> __device__ inline u32 bload_scale(rsrc_t r, u32 voff, int soff) {
  if constexpr (ST == I4_F32) return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
  else return (u32)__builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
}

template <int XT> __device__ inline f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (XT == I4_F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// 8 exact halves M + q of one tile word (nibble slots (p, p + 4) -> half pair p),
// columns 8m .. 8m + 7 in order
template <int XT> __device__ inline u32x4 decode8(u32 w, u32 mg) {
  constexpr u32 MK = 0x000F000Fu;
  return u32x4{(w & MK) | mg, ((w >> 4) & MK) | mg, ((w >> 8) & MK) | mg, ((w >> 12) & MK) | mg};
}

// fp16 pair (M + q0, M + q1) + nz, nz = (-(M + z), -(M + z)): exactly (q0 - z, q1 - z)
__device__ inline u32 sub_zero(u32 p, u32 nz) {
  return __builtin_bit_cast(u32, __builtin_bit_cast(f16x2, p) + __builtin_bit_cast(f16x2, nz));
}

// -(M + z) twice, fp16, for the zero point of group g held in zero word zw
__device__ inline u32 neg_zero2(u32 zw, int g) {
  return (0xE400u | ((zw >> (4 * (g & 7))) & 15u)) * 0x00010001u;
}

// B operand of one MFMA step (nz: neg_zero2 of the step's group, fp16 only;
// mg: magic_v<XT>())
template <int XT> __device__ inline u32x4 b_operand(u32 word, u32 nz, u32 mg) {
  u32x4 b = decode8<XT>(word, mg);
  if constexpr (XT == I4_F16) {
    b.x = sub_zero(b.x, nz);
    b.y = sub_zero(b.y, nz);
    b.z = sub_zero(b.z, nz);
    b.w = sub_zero(b.w, nz);
  }
  return b;
}

// the group scale as two fp16 copies (rounded to fp16 when stored wider)
template <int ST> __device__ inline u32 scale_h2(u32 raw) {
  if constexpr (ST == I4_F16) {
    return (raw & 0xFFFFu) * 0x00010001u;
  } else {
    const u32 h = __builtin_bit_cast(uint16_t, (_Float16)scale_from_raw<ST>(raw));
    return h * 0x00010001u;
  }
}

// fp16 pairs a * s (one v_pk_mul_f16)
__device__ inline u32 mul_h2(u32 a, u32 s) {
  return __builtin_bit_cast(u32, __builtin_bit_cast(f16x2, a) * __builtin_bit_cast(f16x2, s));
}

// fp16 B operand times the group scale: (q - z) s, one rounding per element.
// The components go through scalars: a bit cast applied directly to a vector
// component expression (b.y) reads component 0 with this compiler.
__device__ inline u32x4 scale_b(u32x4 b, u32 s2) {
  const u32 b0 = b.x, b1 = b.y, b2 = b.z, b3 = b.w;
  return u32x4{mul_h2(b0, s2), mul_h2(b1, s2), mul_h2(b2, s2), mul_h2(b3, s2)};
}

// first row block of n-block nb of wave `wave` in column tile `tile`
template <bool GATEUP, int NB>
__device__ inline int nblock(int tile, int wave, int nb, int I) {
  if constexpr (GATEUP)
    return tile * (2 * NB) + (NB / 2) * wave + (nb % (NB / 2)) + (nb >= NB / 2 ? (I >> 4) : 0);
  else
    return tile * (4 * NB) + NB * wave + nb;
}

// the weight operands of one wave: NB n-blocks of expert e, lane (r, j).
// Lane offsets live in VGPRs; the n-block offsets are wave-uniform and go in
// the scalar offset of each load, with the superchunk / group offset.
template <int ST, int NB> struct WBuf {
  rsrc_t p, s, z;
  u32 lw, ls, lz;              // per-lane byte offsets
  int bw[NB], bs[NB], bz[NB];  // per-n-block byte offsets (wave-uniform)
  u32 zor;                     // 0x88888888 when the weight has no zero points
  int gshift;
};

template <int ST, int NB>
__device__ inline WBuf<ST, NB> wbuf(const TW& w, int e, const int (&blk)[NB], int r, int j) {
  constexpr int SB = ST == I4_F32 ? 4 : 2;
  const int SC = w.K >> 7;
  const int NG = (w.K + (32 << w.gshift) - 1) >> (w.gshift + 5), NZW = (NG + 7) >> 3;
  WBuf<ST, NB> b;
  b.p = rsrc(w.packed + e * w.pes, (u32)w.N * (u32)(w.K >> 1));
  b.s = rsrc((const char*)w.scale + e * w.ses * SB, (u32)w.N * NG * SB);
  if (w.zeros) {
    b.z = rsrc(w.zeros + e * w.zes, (u32)w.N * NZW * 4u);
    b.zor = 0u;
  } else {
    b.z = rsrc(w.packed, 0u);
    b.zor = 0x88888888u;
  }
  b.lw = (u32)r * 64u + (u32)j * 16u;
  b.ls = (u32)r * SB;
  b.lz = (u32)r * 4u;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    b.bw[nb] = blk[nb] * SC * 1024;
    b.bs[nb] = blk[nb] * NG * 16 * SB;
    b.bz[nb] = blk[nb] * NZW * 64;
  }
  b.gshift = w.gshift;
  return b;
}

// superchunk sc of every n-block: the 16-byte tile word, the raw scale(s) and
// the zero word (one zero word covers the superchunk's groups).  Nothing here
// touches the loaded values, so issuing never waits for a load.
template <int ST, bool GB, int NB>
__device__ inline void wissue(const WBuf<ST, NB>& b, int sc, TSlot<GB> (&o)[NB]) {
  constexpr int SB = ST == I4_F32 ? 4 : 2;
  const int g0 = (4 * sc) >> b.gshift;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    o[nb].w = bload16(b.p, b.lw, b.bw[nb] + sc * 1024);
    if constexpr (GB) {
      o[nb].s[0] = bload_scale<ST>(b.s, b.ls, b.bs[nb] + g0 * 16 * SB);
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t)
        o[nb].s[t] = bload_scale<ST>(b.s, b.ls, b.bs[nb] + ((4 * sc + t) >> b.gshift) * 16 * SB);
    }
    o[nb].z = bload4(b.z, b.lz, b.bz[nb] + (g0 >> 3) * 64);  // | zor where it is used
  }
}

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

// One entry (<= 16 MB tokens of one expert) x one column tile.  MB m-blocks
// of 16 tokens (1 for the small entries, 4 for the large ones), NB n-blocks
// of 16 weight rows per wave.
// LIN: a dense linear layer (E = 1) over M rows of src: entry blockIdx.y is
// rows [16 MB y, 16 MB (y + 1)) in order (no entry list, no permutation), and
// the epilogue writes y[row][n] + bias[n] in dtype ot to `ys`.  With ksplit >
// 1, blockIdx.z takes the z-th of ksplit contiguous ranges of superchunks and
// writes its fp32 partial sums to part[z][row][n] instead (k_linear_finish
// adds them up).
// The body takes its block coordinates (bx: column tile, by: entry, bz: K range)
// and its LDS (two staging buffers of 16 MB tokens, XSB uint4 apart, and two
// activation-sum buffers, XSUMB floats apart) from the kernel that runs it, so one
// launch can serve entries of both sizes (k_tile_mfma_mixed).
// RING: weight superchunks in flight per wave (2 or 3 register slots).
// HAND (one m-block, not LIN): the two projections share a launch (k_tile_mfma_gd).  The
// gate_up workgroups write act through to memory, every NaN in canonical form; the down
// workgroups read act and, before staging each superchunk, reload it past the L1 until
// no value holds the pending pattern (act was set to it one launch earlier), at most
// max_polls times: then their rows come out NaN and I4_ERR_HANDOFF goes to *status.
// hsrc is act again, without __restrict__, so the reloads stay inside the wait loop.
template <int XT, int ST, bool GB, bool GATEUP, int NB, int MB, bool LIN, int RING = 3,
          bool HAND = false>
__device__ inline void tile_mfma_body(
    int bx, int by, int bz, u32x4* __restrict__ xs0, int XSB, float* __restrict__ xsum0,
    int XSUMB, const uint16_t* __restrict__ src, u32 src_bytes, int topk,
    const int4* __restrict__ entries, const int* __restrict__ n_entries,
    const int32_t* __restrict__ perm, const TW& w, int I, uint16_t* __restrict__ act,
    float* __restrict__ ys, int M, const void* __restrict__ bias, int ot, int ksplit,
    float* __restrict__ part, const uint16_t* hsrc = nullptr, int max_polls = 0,
    int32_t* __restrict__ status = nullptr) {
  static_assert(!HAND || (MB == 1 && !LIN), "the hand-over serves one-m-block entries");
  constexpr bool EXACT = XT == I4_F16;
  // fp16 with several m-blocks folds the scale into B (see the top); one
  // m-block keeps the exact form, whose extra registers fit its occupancy
  constexpr bool FOLD = EXACT && MB > 1;
  constexpr int COLS = GATEUP ? 32 * NB : 64 * NB;
  constexpr int TOK = 16 * MB;
  static_assert(!GATEUP || NB % 2 == 0, "gate_up pairs gate and up blocks");
  static_assert(MB == 1 || MB == 4 || MB == 8, "staging maps 256 threads onto 16, 64 or 128 tokens");
  // 128-token tiles stage one superchunk at a time (the LDS of two would halve occupancy)
  constexpr bool DBUF = MB <= 4;
  static_assert(!(LIN && GATEUP), "a linear layer is a plain projection");
  auto XS = [&](int buf, int i) -> u32x4& { return xs0[buf * XSB + i]; };
  auto XSUM = [&](int buf, int i) -> float& { return xsum0[buf * XSUMB + i]; };
  if (!LIN && by >= *n_entries) return;
  const u32 mg = magic_v<XT>();
  const int4 en = LIN ? int4{0, by * TOK, min(TOK, M - by * TOK), 0} : entries[by];
  const int e = en.x, pos0 = en.y, cnt = en.z;
  const int K = w.K, SC_ALL = K >> 7;
  // superchunks [scb, scb + SC) of this workgroup (all of them unless split)
  const int scb = LIN ? (bz * SC_ALL) / ksplit : 0;
  const int SC = LIN ? ((bz + 1) * SC_ALL) / ksplit - scb : SC_ALL;
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, ln = lane & 15, kb = lane >> 4;
  const bool ev = (unsigned)e < (unsigned)w.E;
  const int nmb = MB == 1 ? 1 : (cnt + 15) >> 4;
  int blk[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) blk[nb] = nblock<GATEUP, NB>(bx, wave, nb, I);
  const WBuf<ST, NB> wb = wbuf<ST, NB>(w, ev ? e : 0, blk, ln, kb);
  // staging role: token tid / (16 / MB), words MB (tid % (16 / MB)) .. + MB - 1 of its
  // 16 (MB = 1: one word; 4: one chunk; 8: two chunks)
  constexpr int WPT = MB;  // 16-byte words per thread and superchunk
  constexpr int TPT = 16 / MB;  // threads per staged token
  const int tk = (int)threadIdx.x / TPT;
  const int kw = MB * ((int)threadIdx.x % TPT);  // first word
  const int row = GATEUP ? perm[pos0 + min(tk, cnt - 1)] / topk : pos0 + min(tk, cnt - 1);
  const rsrc_t xr = rsrc(src, src_bytes);
  const u32 vx = ((u32)row * (u32)K + 8u * (u32)kw) * 2u;
  // Ring slot: the weights of one superchunk and (XR) its activation words too, issued
  // right after the weights: the in-order wait for them at staging time then only covers
  // loads the step needs anyway.  Two-slot rings carry them (one word per thread for one
  // m-block, four for the large entries of the mixed launch: two superchunks of lead, 118
  // VGPRs); the three-slot ring of the other multi-m-block forms loads them one step ahead
  // instead (three slots of four words would cost occupancy).  Measured on the M=512
  // layer: 118.9 / 119.4 -> 117.5 / 116.5 us for the large entries' two-slot form.
  constexpr bool XR = MB == 1 || RING == 2;
  struct Slot {
    TSlot<GB> w[NB];
    u32x4 x[XR ? WPT : 1];
  };
  u32x4 xd[WPT];
  const rsrc_t hr = rsrc(HAND && !GATEUP ? hsrc : src, src_bytes);
  // HAND down reads act through the caches first (an entry's activations are read by
  // every column tile of it); only a word that still holds the pending pattern, in memory
  // or in a line the L2 took before its producer wrote it, is reloaded past them (wait_x)
  auto load_x = [&](int sc, u32x4* dst) {
    sc = scb + min(sc, SC - 1);
#pragma unroll
    for (int q = 0; q < WPT; ++q) dst[q] = bload16(xr, vx + 16u * q, sc * 256);
  };
  // HAND down: reload superchunk sc's activation word until no thread holds a pending
  // value (the workgroup decides together, so every thread runs the same passes)
  bool late = false;
  auto wait_x = [&](int sc, u32x4& x) {
    sc = scb + min(sc, SC - 1);
    for (int it = 0;; ++it) {
      if (!__syncthreads_or(has_pending(x))) return;
      if (it >= max_polls) {
        late = true;
        return;
      }
      __builtin_amdgcn_s_sleep(1);
      asm volatile("" ::: "memory");
      x = bload16_coherent(hr, vx, sc * 256);
    }
  };
  auto commit_x = [&](int buf, const u32x4* src_x) {
    float sm = 0.f, sm1 = 0.f;  // sm1: the second chunk of a two-chunk thread (MB = 8)
#pragma unroll
    for (int q = 0; q < WPT; ++q) {
      XS(buf, xs_at(tk, kw + q)) = src_x[q];
      if constexpr (!EXACT) {
        if (q < 4) sm += sum8<XT>(src_x[q]).y;
        else sm1 += sum8<XT>(src_x[q]).y;
      }
    }
    if constexpr (!EXACT) {
      if constexpr (MB == 1) {
        sm = group_sum<4>(sm);  // the chunk's 4 words sit in 4 adjacent lanes
        if ((kw & 3) == 0) XSUM(buf, 4 * tk + (kw >> 2)) = sm;
      } else if constexpr (MB == 4) {
        XSUM(buf, 4 * tk + (kw >> 2)) = sm;
      } else {  // two chunks per thread
        XSUM(buf, 4 * tk + (kw >> 2)) = sm;
        XSUM(buf, 4 * tk + (kw >> 2) + 1) = sm1;
      }
    }
  };
  auto issue = [&](int sc, Slot& sl) {
    wissue<ST, GB, NB>(wb, scb + min(sc, SC - 1), sl.w);
    if constexpr (XR) load_x(sc, sl.x);
  };
  f32x4 res[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) res[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  // S of rows 16 mb + 4 j + i over chunks [t0, t0 + nt) of the staged superchunk
  auto rows_sum = [&](int buf, int mb, int t0, int nt, float (&sm)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float* p = &XSUM(buf, 4 * (16 * mb + 4 * kb + i));
      float v = 0.f;
      for (int t = t0; t < t0 + nt; ++t) v += p[t];
      sm[i] = v;
    }
  };
  auto compute = [&](int sc, const TSlot<GB> (&sl)[NB], int buf) {
    const int g0 = (4 * sc) >> w.gshift;
    u32 zw[NB], nz[NB];  // zero words; GB: one zero point for the superchunk
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      zw[nb] = sl[nb].z | wb.zor;
      nz[nb] = EXACT && GB ? neg_zero2(zw[nb], g0) : 0u;
    }
    if constexpr (FOLD) {
      // fp16, several m-blocks: B = (q - z) s, one rounding, accumulated
      // straight into res
      u32 s2[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) s2[nb] = GB ? scale_h2<ST>(sl[nb].s[0]) : 0u;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int g = (4 * sc + t) >> w.gshift;
        auto bop = [&](int nb) {
          const u32 z2 = GB ? nz[nb] : neg_zero2(zw[nb], g);
          const u32 sc2 = GB ? s2[nb] : scale_h2<ST>(sl[nb].s[t]);
          return scale_b(b_operand<XT>(word_t(sl[nb].w, t), z2, mg), sc2);
        };
        if constexpr (MB == 1) {  // one m-block: each B operand feeds one MFMA
          const u32x4 a = XS(buf, xs_at(ln, 4 * t + kb));
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) res[0][nb] = mfma16<XT>(a, bop(nb), res[0][nb]);
        } else {
          u32x4 b[NB];
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) b[nb] = bop(nb);
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) {
            if (mb < nmb) {
              const u32x4 a = XS(buf, xs_at(16 * mb + ln, 4 * t + kb));
#pragma unroll
              for (int nb = 0; nb < NB; ++nb) res[mb][nb] = mfma16<XT>(a, b[nb], res[mb][nb]);
            }
          }
        }
      }
      return;
    } else {
    // exact: B = q - z (fp16) or M + q (bf16), per-group correction (bf16 with
    // the activation sums)
    f32x4 d[MB][NB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) d[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int g = (4 * sc + t) >> w.gshift;
      if constexpr (MB == 1) {  // one m-block: each B operand feeds one MFMA
        const u32x4 a = XS(buf, xs_at(ln, 4 * t + kb));
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          d[0][nb] = mfma16<XT>(
              a, b_operand<XT>(word_t(sl[nb].w, t), GB ? nz[nb] : neg_zero2(zw[nb], g), mg),
              d[0][nb]);
      } else {
        u32x4 b[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          b[nb] = b_operand<XT>(word_t(sl[nb].w, t), GB ? nz[nb] : neg_zero2(zw[nb], g), mg);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          if (mb < nmb) {
            const u32x4 a = XS(buf, xs_at(16 * mb + ln, 4 * t + kb));
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) d[mb][nb] = mfma16<XT>(a, b[nb], d[mb][nb]);
          }
        }
      }
      if constexpr (!GB) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          if (mb < nmb) {
            float sm[4] = {0.f, 0.f, 0.f, 0.f};
            if constexpr (!EXACT) rows_sum(buf, mb, t, 1, sm);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
              correct<XT, ST>(res[mb][nb], d[mb][nb], sl[nb].s[t], zw[nb], g, sm);
              d[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
          }
        }
      }
    }
    if constexpr (GB) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        if (mb < nmb) {
          float sm[4] = {0.f, 0.f, 0.f, 0.f};
          if constexpr (!EXACT) rows_sum(buf, mb, 0, 4, sm);
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            correct<XT, ST>(res[mb][nb], d[mb][nb], sl[nb].s[0], zw[nb], g0, sm);
        }
      }
    }
    }
  };
  // one superchunk: stage its activations (loaded one step earlier), load the
  // next step's, multiply, refill this weight slot three superchunks ahead.
  // Staging and barrier run past the last superchunk too (clamped data that
  // nothing reads): a staging store inside the guard would let the compiler
  // sink the activation load down to it and lose the prefetch.
  auto step = [&](int sc, Slot& sl) {
    const int buf = DBUF ? sc & 1 : 0;
    if constexpr (!DBUF) __syncthreads();  // the previous superchunk's reads are done
    if constexpr (XR) {
      if constexpr (HAND && !GATEUP) wait_x(sc, sl.x[0]);
      commit_x(buf, sl.x);
    } else {
      commit_x(buf, xd);
    }
    __syncthreads();
    if constexpr (!XR) load_x(sc + 1, xd);  // unconditional (clamped), like every load
    if (sc < SC) compute(scb + sc, sl.w, buf);
    issue(sc + RING, sl);
  };
  // Prologue loads in ring order, first turn peeled: the activation loads wait
  // for perm and land after the weights, and a loop header reached from the
  // prologue as well would wait for nearly every load in flight.
  static_assert(RING == 2 || RING == 3, "two or three ring slots");
  if constexpr (RING == 3) {
    Slot s0, s1, s2;
    issue(0, s0);
    __builtin_amdgcn_sched_barrier(0);
    issue(1, s1);
    __builtin_amdgcn_sched_barrier(0);
    issue(2, s2);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (!XR) load_x(0, xd);
    __builtin_amdgcn_sched_barrier(0);
    step(0, s0);
    step(1, s1);
    step(2, s2);
    for (int sc = 3; sc < SC; sc += 3) {
      step(sc, s0);
      step(sc + 1, s1);
      step(sc + 2, s2);
    }
  } else {
    Slot s0, s1;
    issue(0, s0);
    __builtin_amdgcn_sched_barrier(0);
    issue(1, s1);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (!XR) load_x(0, xd);
    __builtin_amdgcn_sched_barrier(0);
    step(0, s0);
    step(1, s1);
    for (int sc = 2; sc < SC; sc += 2) {
      step(sc, s0);
      step(sc + 1, s1);
    }
  }
  // epilogue: lane holds rows m = 16 mb + 4 j + i of column r.  HAND gate_up gathers the
  // workgroup's 16 x COLS values in LDS and writes each token's row through as 16-byte
  // stores (2-byte write-through stores per lane reached the down workgroups later)
  __shared__ __align__(16) uint16_t s_act[HAND && GATEUP ? 16 * COLS : 8];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 16 * mb + 4 * kb + i;
      if (m < cnt) {
        if constexpr (GATEUP) {
#pragma unroll
          for (int nb = 0; nb < NB / 2; ++nb) {
            const int n = bx * COLS + 16 * (NB / 2) * wave + 16 * nb + ln;
            const float v =
                ev ? silu(res[mb][nb][i]) * res[mb][nb + NB / 2][i] : __builtin_nanf("");
            if constexpr (HAND)
              s_act[m * COLS + (n - bx * COLS)] = v != v ? Half<XT>::QNAN : Half<XT>::from_f32(v);
            else
              act[(int64_t)(pos0 + m) * I + n] = Half<XT>::from_f32(v);
          }
        } else if constexpr (LIN) {
          const int n0 = bx * COLS + 16 * NB * wave + ln;
          const int64_t o = (int64_t)(pos0 + m) * w.N + n0;
          if (ksplit > 1) {
            float* pz = part + (int64_t)bz * M * w.N;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) pz[o + 16 * nb] = res[mb][nb][i];
            continue;
          }
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            const int n = n0 + 16 * nb;
            float v = res[mb][nb][i];
            if (ot == I4_F32) {
              if (bias) v += ((const float*)bias)[n];
              store_out<I4_F32>(ys, o + 16 * nb, v);
            } else if (ot == I4_F16) {
              if (bias) v += Half<I4_F16>::to_f32(((const uint16_t*)bias)[n]);
              store_out<I4_F16>(ys, o + 16 * nb, v);
            } else {
              if (bias) v += Half<I4_BF16>::to_f32(((const uint16_t*)bias)[n]);
              store_out<I4_BF16>(ys, o + 16 * nb, v);
            }
          }
        } else {
          const int64_t o = (int64_t)perm[pos0 + m] * w.N + bx * COLS + 16 * NB * wave + ln;
#pragma unroll
          // the expert's output in the activation dtype (k_moe_combine sums the slots)
          for (int nb = 0; nb < NB; ++nb)
            ((uint16_t*)ys)[o + 16 * nb] =
                Half<XT>::from_f32(ev && !late ? res[mb][nb][i] : __builtin_nanf(""));
        }
      }
    }
  }
  if constexpr (HAND && GATEUP) {
    constexpr int WPR = COLS / 8;  // 16-byte words per token row
    __syncthreads();
    const int m = (int)threadIdx.x / WPR, q = (int)threadIdx.x % WPR;
    if (m < cnt) {
      const rsrc_t r = rsrc(act + (int64_t)(pos0 + m) * I + bx * COLS, (u32)COLS * 2u);
      __builtin_amdgcn_raw_buffer_store_b128(((const u32x4*)s_act)[m * WPR + q], r, (u32)q * 16u,
                                             0, kCoherent);
    }
  }
  if constexpr (HAND && !GATEUP)  // a wait that gave up is reported (status nullable)
    if (late && status && threadIdx.x == 0) *status = I4_ERR_HANDOFF;
}

// WPE: minimum waves per SIMD the register allocation must allow (1: no bound).  The
// one-m-block down projection on fp16 activations with one group per superchunk fits
// eight (64 VGPRs, no spill; the other forms would spill), so all of a T <= 64 down
// launch's workgroups are resident at once.
template <int XT, int ST, bool GB, bool GATEUP, int NB, int MB, bool LIN = false, int WPE = 1>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE))) void k_tile_mfma(
    const uint16_t* __restrict__ src, u32 src_bytes, int topk, const int4* __restrict__ entries,
    const int* __restrict__ n_entries, const int32_t* __restrict__ perm, TW w, int I,
    uint16_t* __restrict__ act, float* __restrict__ ys, int M = 0,
    const void* __restrict__ bias = nullptr, int ot = 0, int ksplit = 1,
    float* __restrict__ part = nullptr) {
  constexpr int TOK = 16 * MB;
  constexpr int NBUF = MB <= 4 ? 2 : 1;  // 128-token tiles are staged single-buffered
  __shared__ u32x4 xs[NBUF][TOK * MF_TSTRIDE];
  __shared__ float xsum[NBUF][TOK * 4];  // bf16: per token and chunk
  // one-m-block entries alone: two ring slots keep the wave at <= 80 VGPRs, so six
  // workgroups fit a CU and the T <= 64 launches run in one round
  tile_mfma_body<XT, ST, GB, GATEUP, NB, MB, LIN, (MB == 1 && !LIN) ? 2 : 3>(
      blockIdx.x, blockIdx.y, blockIdx.z, &xs[0][0], TOK * MF_TSTRIDE, &xsum[0][0], TOK * 4, src,
      src_bytes, topk, entries, n_entries, perm, w, I, act, ys, M, bias, ot, ksplit, part);
}

// Both entry lists of a projection in one launch: rows [0, n_large) of the grid
// take the large entries (four m-blocks), the next n_small rows the small ones
// (one m-block) and the rest of the grid (sized for the worst case) exits.  The
// large ones come first, so the longest workgroups are dispatched first and the
// small entries' weight streaming fills the machine behind them; the idle rows
// come last, so no small entry waits behind their dispatch.
template <int XT, int ST, bool GB, bool GATEUP, int NB>
__global__ __launch_bounds__(256) void k_tile_mfma_mixed(
    const uint16_t* __restrict__ src, u32 src_bytes, int topk, const int4* __restrict__ large,
    const int* __restrict__ n_large, const int4* __restrict__ small,
    const int* __restrict__ n_small, const int32_t* __restrict__ perm, TW w, int I,
    uint16_t* __restrict__ act, float* __restrict__ ys) {
  constexpr int TOKL = MF_TOK;
  constexpr int NBUF = MF_TOK <= 64 ? 2 : 1;  // 128-token tiles are staged single-buffered
  __shared__ u32x4 xs[NBUF * TOKL * MF_TSTRIDE];
  __shared__ float xsum[NBUF * TOKL * 4];
  const int y = blockIdx.y, nl = *n_large;
  if (y < nl)
    tile_mfma_body<XT, ST, GB, GATEUP, NB, MF_TOK / 16, false, 2>(
        blockIdx.x, y, 0, xs, TOKL * MF_TSTRIDE, xsum, TOKL * 4, src, src_bytes,
        topk, large, n_large, perm, w, I, act, ys, 0, nullptr, 0, 1, nullptr);
  else
    tile_mfma_body<XT, ST, GB, GATEUP, NB, 1, false>(
        blockIdx.x, y - nl, 0, xs, 16 * MF_TSTRIDE, xsum, 16 * 4, src,
        src_bytes, topk, small, n_small, perm, w, I, act, ys, 0, nullptr, 0, 1, nullptr);
}

// Both projections of the small entries in one launch (T <= 64, every expert in entries
// of <= 16 tokens): blocks [0, n_gu) are the gate_up workgroups (column tile b % gu_cols of
// entry b / gu_cols), the later blocks the down workgroups (column tile d % dn_cols of
// entry d / dn_cols), which stream their first weight superchunks at once and take each
// superchunk of their entry's act over as its gate_up workgroups write it through (act
// holds the pending pattern before the launch).  Only later blocks wait, and only for
// earlier ones.  WPE: waves per SIMD the register allocation must allow; fp16 with one
// group per superchunk fits six (80 VGPRs, no spill; 104 unbounded), the other forms
// would spill and run unbounded.
// block b -> (down?, entry, column tile): every gate_up block (n_e entries x gu_cols
// tiles), then every down block; down_only: the down blocks alone.  (Interleaving chunks
// of entries -- gate_up of chunk c, then down of chunk c - 1 -- measured slower, 74.7-79.9
// against 70.2-70.6 us per M = 32 layer for chunks of 32 to 8 entries: the waiting down
// workgroups hold slots the gate_up stream needs.)
__device__ inline void gd_map(int b, int n_e, int gu_cols, int dn_cols, int down_only, bool& dn,
                              int& e, int& tile) {
  dn = down_only || b >= gu_cols * n_e;
  const int r = dn && !down_only ? b - gu_cols * n_e : b;
  const int c = dn ? dn_cols : gu_cols;
  e = r / c;
  tile = r % c;
}

template <int XT, int ST, bool GB, int NB, int WPE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE))) void k_tile_mfma_gd(
    const uint16_t* __restrict__ x, u32 x_bytes, int topk, const int4* __restrict__ ent,
    const int* __restrict__ nent, const int32_t* __restrict__ perm, TW wg, TW wd, int I,
    uint16_t* act, u32 act_bytes, float* __restrict__ ys, int n_e, int gu_cols, int dn_cols,
    int down_only, int max_polls, int32_t* __restrict__ status) {
  __shared__ u32x4 xs[2 * 16 * MF_TSTRIDE];
  __shared__ float xsum[2 * 16 * 4];
  bool dn;
  int e, tile;
  gd_map((int)blockIdx.x, n_e, gu_cols, dn_cols, down_only, dn, e, tile);
  if (!dn) {
    tile_mfma_body<XT, ST, GB, true, NB, 1, false, 2, true>(
        tile, e, 0, xs, 16 * MF_TSTRIDE, xsum, 16 * 4, x, x_bytes, topk, ent, nent, perm, wg, I,
        act, nullptr, 0, nullptr, 0, 1, nullptr);
  } else {
    tile_mfma_body<XT, ST, GB, false, NB, 1, false, 2, true>(
        tile, e, 0, xs, 16 * MF_TSTRIDE, xsum, 16 * 4, act, act_bytes, 0, ent, nent, perm, wd, 0,
        nullptr, ys, 0, nullptr, 0, 1, nullptr, act, max_polls, status);
  }
}

// ---------------------------------------------------------------------------
template <int XT, int ST, bool GB, bool GATEUP>
static int mfma_t(bool small, int max_entries, const void* src, int src_rows, int topk,
                  const int4* ent, const int* nent, const int32_t* perm, const TW& w, int I,
                  void* act, float* ys, hipStream_t s) {
  const int64_t src_bytes = (int64_t)src_rows * w.K * 2;
  // buffer offsets are 32-bit: the activation rows and one expert's weights must fit
  if (src_bytes >= ((int64_t)1 << 31) || (int64_t)w.N * w.K / 2 >= ((int64_t)1 << 31))
    return I4_ERR_SHAPE;
  const int n_out = GATEUP ? I : w.N;
  const int cols = GATEUP ? 32 * MF_NB : 64 * MF_NB;
#define I4_MF_LAUNCH(NB_, MB_)                                                                  \
  hipLaunchKernelGGL((k_tile_mfma<XT, ST, GB, GATEUP, NB_, MB_, false,                         \
                                  (!GATEUP && MB_ == 1 && XT == I4_F16 && GB) ? 8 : 1>),       \
                     dim3(n_out / (cols * NB_ / MF_NB), max_entries), dim3(256), 0, s,          \
                     (const uint16_t*)src, (u32)src_bytes, topk, ent, nent, perm, w, I,         \
                     (uint16_t*)act, ys)
  // small entries: one m-block; MF_NB n-blocks per wave (twice the n-blocks, half the
  // workgroups, was 5 % slower per M = 32 layer and 2 % per M = 512 layer)
  if (small) I4_MF_LAUNCH(MF_NB, 1);
  else I4_MF_LAUNCH(MF_NB, MF_TOK / 16);
#undef I4_MF_LAUNCH
  return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;
}

template <int XT, int ST>
int launch_mfma_gate_up(bool small, int max_entries, const void* x, int T, int topk,
                        const int4* ent, const int* nent, const int32_t* perm, const TW& w, int I,
                        void* act, hipStream_t s) {
  if (w.gshift >= 2)
    return mfma_t<XT, ST, true, true>(small, max_entries, x, T, topk, ent, nent, perm, w, I, act,
                                      nullptr, s);
  return mfma_t<XT, ST, false, true>(small, max_entries, x, T, topk, ent, nent, perm, w, I, act,
                                     nullptr, s);
}

template <int XT, int ST>
int launch_mfma_down(bool small, int max_entries, const void* act, int rows, const int4* ent,
                     const int* nent, const int32_t* perm, const TW& w, void* ys, hipStream_t s) {
  // the kernel's output pointer is typed for the dense linear's fp32 path; the
  // MoE down projection stores activation-dtype halves through it
  if (w.gshift >= 2)
    return mfma_t<XT, ST, true, false>(small, max_entries, act, rows, 0, ent, nent, perm, w, 0,
                                       nullptr, (float*)ys, s);
  return mfma_t<XT, ST, false, false>(small, max_entries, act, rows, 0, ent, nent, perm, w, 0,
                                      nullptr, (float*)ys, s);
}

template <int XT, int ST>
int launch_mfma_gd(int max_entries, const void* x, int T, int topk, const int4* ent,
                   const int* nent, const int32_t* perm, const TW& wg, const TW& wd, int I,
                   void* act, void* ys, int32_t* status, int max_polls, bool down_only,
                   hipStream_t s) {
  const int64_t x_bytes = (int64_t)T * wg.K * 2, act_bytes = (int64_t)T * topk * I * 2;
  if (act_bytes >= ((int64_t)1 << 31) || (int64_t)wg.N * wg.K / 2 >= ((int64_t)1 << 31) ||
      (int64_t)wd.N * wd.K / 2 >= ((int64_t)1 << 31))
    return I4_ERR_SHAPE;
  if (wg.gshift != wd.gshift) return I4_ERR_SHAPE;  // one group size for both
  const int gu_cols = I / (32 * MF_NB), dn_cols = wd.N / (64 * MF_NB);
  // down_only: the down workgroups alone (their waits then give up after max_polls)
  const dim3 grid((down_only ? 0 : gu_cols * max_entries) + dn_cols * max_entries);
#define I4_GD_LAUNCH(GB_)                                                                     \
  hipLaunchKernelGGL((k_tile_mfma_gd<XT, ST, GB_, MF_NB, (XT == I4_F16 && GB_) ? 6 : 1>),     \
                     grid, dim3(256), 0, s,                                                   \
                     (const uint16_t*)x, (u32)x_bytes, topk, ent, nent, perm, wg, wd, I,      \
                     (uint16_t*)act, (u32)act_bytes, (float*)ys, max_entries, gu_cols,       \
                     dn_cols,                                                                 \
                     (int)down_only, max_polls, status)
  if (wg.gshift >= 2) I4_GD_LAUNCH(true);
  else I4_GD_LAUNCH(false);
#undef I4_GD_LAUNCH
  return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;
}

// both entry lists of one projection in one launch (k_tile_mfma_mixed)
template <int XT, int ST, bool GB, bool GATEUP>
static int mixed_t(int max_large, int max_small, const void* src, int src_rows, int topk,
                   const int4* large, const int* n_large, const int4* small, const int* n_small,
                   const int32_t* perm, const TW& w, int I, void* act, void* ys, hipStream_t s) {
  const int64_t src_bytes = (int64_t)src_rows * w.K * 2;
  if (src_bytes >= ((int64_t)1 << 31) || (int64_t)w.N * w.K / 2 >= ((int64_t)1 << 31))
    return I4_ERR_SHAPE;
  const int n_out = GATEUP ? I : w.N;
  const int cols = GATEUP ? 32 * MF_NB : 64 * MF_NB;
  hipLaunchKernelGGL((k_tile_mfma_mixed<XT, ST, GB, GATEUP, MF_NB>),
                     dim3(n_out / cols, max_large + max_small), dim3(256), 0, s,
                     (const uint16_t*)src, (u32)src_bytes, topk, large, n_large, small, n_small,
                     perm, w, I, (uint16_t*)act, (float*)ys);
  return hipGetLastError() == hipSuccess ? I4_OK : I4_ERR_LAUNCH;
}

template <int XT, int ST>
int launch_mfma_mixed(bool gate_up, int max_large, int max_small, const void* src, int src_rows,
                      int topk, const int4* large, const int* n_large, const int4* small,
                      const int* n_small, const int32_t* perm, const TW& w, int I, void* out,
                      hipStream_t s) {
  // gate_up: src = x [T][H], out = act; down: src = act [rows][I], out = ys
  const bool gb = w.gshift >= 2;
  if (gate_up)
    return gb ? mixed_t<XT, ST, true, true>(max_large, max_small, src, src_rows, topk, large,
                                            n_large, small, n_small, perm, w, I, out, nullptr, s)
              : mixed_t<XT, ST, false, true>(max_large, max_small, src, src_rows, topk, large,
                                             n_large, small, n_small, perm, w, I, out, nullptr, s);
  return gb ? mixed_t<XT, ST, true, false>(max_large, max_small, src, src_rows, 0, large, n_large,
                                           small, n_small, perm, w, 0, nullptr, out, s)
            : mixed_t<XT, ST, false, false>(max_large, max_small, src, src_rows, 0, large,
                                            n_large, small, n_small, perm, w, 0, nullptr, out, s);
}

// y[r][n] = sum_z part[z][r][n] + bias[n] in dtype ot, the K ranges in order
__global__ __launch_bounds__(256) void k_linear_finish(const float* __restrict__ part, int ksplit,
                                                       int64_t total, int N,
                                                       const void* __restrict__ bias,
                                                       void* __restrict__ y, int ot) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  float v = 0.f;
  for (int z = 0; z < ksplit; ++z) v += part[z * total + i];
  const int n = (int)(i % N);
  if (ot == I4_F32) {
    if (bias) v += ((const float*)bias)[n];
    store_out<I4_F32>(y, i, v);
  } else if (ot == I4_F16) {
    if (bias) v += Half<I4_F16>::to_f32(((const uint16_t*)bias)[n]);
    store_out<I4_F16>(y, i, v);
  } else {
    if (bias) v += Half<I4_BF16>::to_f32(((const uint16_t*)bias)[n]);
    store_out<I4_BF16>(y, i, v);
  }
}

// K ranges of a dense linear launch: a grid of fewer than 256 output tiles
// (few rows or few columns) is split along K until it has about 512
// workgroups, each range keeping at least 4 superchunks
int linear_ksplit(int M, int N, int K) {
  const int tiles = (N / (64 * MF_NB)) * ((M + LIN_TOK - 1) / LIN_TOK);
  const int sc = K / 128;
  if (tiles >= 256 || sc < 8) return 1;
  int ks = (512 + tiles - 1) / tiles;
  if (ks > sc / 4) ks = sc / 4;
  return ks < 1 ? 1 : ks;
}

size_t linear_tile_workspace_bytes(int M, int N, int K) {
  const int ks = linear_ksplit(M, N, K);
  return ks > 1 ? (size_t)ks * M * N * sizeof(float) : 0;
}

// dense linear layer y = x W^T (+ bias), W one tile-layout weight (E = 1),
// x [M][K]: entries of 16 MB rows in order, split along K when the grid is small
template <int XT, int ST>
int launch_mfma_linear(const void* x, int M, const TW& w, const void* bias, void* y, int ot,
                       void* ws, size_t ws_bytes, hipStream_t s) {
  const int64_t src_bytes = (int64_t)M * w.K * 2;
  if (src_bytes >= ((int64_t)1 << 31) || (int64_t)w.N * w.K / 2 >= ((int64_t)1 << 31))
    return I4_ERR_SHAPE;
  constexpr int COLS = 64 * MF_NB, TOK = LIN_TOK;
  if (w.N % COLS != 0 || w.K % 128 != 0 || w.E != 1) return I4_ERR_SHAPE;
  const int ks = linear_ksplit(M, w.N, w.K);
  if (ks > 1 && (!ws || ws_bytes < linear_tile_workspace_bytes(M, w.N, w.K)))
    return I4_ERR_WORKSPACE;
  const dim3 grid(w.N / COLS, (M + TOK - 1) / TOK, ks);
#define I4_LIN(GB_)                                                                            \
  hipLaunchKernelGGL((k_tile_mfma<XT, ST, GB_, false, MF_NB, TOK / 16, true>), grid, dim3(256), \
                     0, s, (const uint16_t*)x, (u32)src_bytes, 0, nullptr, nullptr, nullptr, w, \
                     0, nullptr, (float*)y, M, bias, ot, ks, (float*)ws)
  if (w.gshift >= 2) I4_LIN(true);
  else I4_LIN(false);
#undef I4_LIN
  if (hipGetLastError() != hipSuccess) return I4_ERR_LAUNCH;
  if (ks > 1) {
    const int64_t total = (int64_t)M * w.N;
    hipLaunchKernelGGL(k_linear_finish, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                       (const float*)ws, ks, total, w.N, bias, y, ot);
    if (hipGetLastError() != hipSuccess) return I4_ERR_LAUNCH;
  }
  return I4_OK;
}

#define I4_INST(XT_, ST_)                                                                      \
  template int launch_mfma_linear<XT_, ST_>(const void*, int, const TW&, const void*, void*,   \
                                            int, void*, size_t, hipStream_t);                  \
  template int launch_mfma_gate_up<XT_, ST_>(bool, int, const void*, int, int, const int4*,    \
                                             const int*, const int32_t*, const TW&, int, void*, \
                                             hipStream_t);                                     \
  template int launch_mfma_down<XT_, ST_>(bool, int, const void*, int, const int4*,            \
                                          const int*, const int32_t*, const TW&, void*,        \
                                          hipStream_t);                                        \
  template int launch_mfma_mixed<XT_, ST_>(bool, int, int, const void*, int, int, const int4*, \
                                           const int*, const int4*, const int*, const int32_t*, \
                                           const TW&, int, void*, hipStream_t);                \
  template int launch_mfma_gd<XT_, ST_>(int, const void*, int, int, const int4*, const int*,   \
                                        const int32_t*, const TW&, const TW&, int, void*, void*, \
                                        int32_t*, int, bool, hipStream_t);
I4_INST(I4_F16, I4_F32) I4_INST(I4_F16, I4_F16) I4_INST(I4_F16, I4_BF16)
I4_INST(I4_BF16, I4_F32) I4_INST(I4_BF16, I4_F16) I4_INST(I4_BF16, I4_BF16)
#undef I4_INST

}  // namespace i4
