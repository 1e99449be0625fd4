// Device helpers of the MoE kernels, which read weights in I4_LAYOUT_TILE.
//
// A tile is 16 weight rows x one 128-column superchunk (four 32-column
// chunks): 1 KB.  Lane (r, j) of a wavefront -- r = lane % 16 the row, j =
// lane / 16 the k-group -- loads one 16-byte word holding word j (columns
// 8j..8j+7) of each of the four chunks, so the 64 lanes read the tile's 1 KB
// as one contiguous block.  Component t of that word belongs to chunk 4s + t.
// Nibble slots (i, i + 4) of a word hold the adjacent columns (2i, 2i + 1), so
// the half pairs the decode builds line up with the activations in their
// natural order and no operand needs permuting.
// Scales and zero words are stored per 16-row block and group with the 16
// rows adjacent, so lane r's side loads are coalesced as well.
//
// Groups: GB (group >= 128, a multiple of the superchunk) means one scale and
// zero point per superchunk and one correction after the four chunks; !GB
// (group 32 or 64) takes one scale per chunk and corrects after every chunk.
// Either way each correction covers exactly one group, so every product is
// exact and the sums are fp32.
#pragma once

#include "i4_common.h"

namespace i4 {

struct TW {  // device view of one I4_LAYOUT_TILE weight
  const int32_t* packed;
  const void* scale;
  const int32_t* zeros;
  int64_t pes, ses, zes;  // element strides between experts
  int gshift, E, N, K;
};

// lane (r, j) of row block b of expert e
struct TileRow {
  const u32x4* p;  // superchunk s at p[64 s]
  const void* s;   // scale of group g at element 16 g
  const u32* z;    // zero word of group g at z[zs * (g >> 3)]
  int zs;          // 16, or 0 for the symmetric table
};

template <int ST> __device__ inline TileRow tile_row(const TW& w, int e, int b, int r, int j) {
  const int SC = w.K >> 7;
  const int NG = (w.K + (32 << w.gshift) - 1) >> (w.gshift + 5), NZW = (NG + 7) >> 3;
  TileRow t;
  t.p = (const u32x4*)(w.packed + e * w.pes) + ((int64_t)b * SC * 16 + r) * 4 + j;
  t.s = scale_at<ST>(w.scale, e * w.ses + (int64_t)b * NG * 16 + r);
  if (w.zeros) {
    t.z = (const u32*)w.zeros + e * w.zes + (int64_t)b * NZW * 16 + r;
    t.zs = 16;
  } else {
    t.z = kSymZeros;
    t.zs = 0;
  }
  return t;
}

// one lane's part of one superchunk: the 16-byte word, raw scales (s[0] only
// when GB) and the zero word (one covers the superchunk's groups)
template <bool GB> struct TSlot {
  u32x4 w;
  u32 s[GB ? 1 : 4];
  u32 z;
};

template <int ST, bool GB>
__device__ inline TSlot<GB> tile_load(const TileRow& r, int s, int gshift) {
  TSlot<GB> o;
  o.w = r.p[64 * s];
  if constexpr (GB) {
    o.s[0] = load_scale_raw<ST>(r.s, (int64_t)16 * ((4 * s) >> gshift));
  } else {
#pragma unroll
    for (int t = 0; t < 4; ++t) o.s[t] = load_scale_raw<ST>(r.s, (int64_t)16 * ((4 * s + t) >> gshift));
  }
  o.z = r.z[r.zs * (((4 * s) >> gshift) >> 3)];
  return o;
}

__device__ inline u32 word_t(const u32x4& w, int t) {
  return t == 0 ? w.x : t == 1 ? w.y : t == 2 ? w.z : w.w;
}

// zero point of group g from the zero word of its 8-group block
__device__ inline float zero_of(u32 zw, int g) { return (float)((zw >> (4 * (g & 7))) & 15u); }

// Activation staging for the decode kernels: nr rows of K halves in LDS, word
// jw of chunk c of row r at xs[(4 r + jw) C + c] in natural order, and
// its (Sb, S) at sums[(4 r + jw) C + c] (one entry per 16-byte word: a lane
// of a tile covers one word of each chunk).  issue() puts up to 4 loads per
// thread in flight and returns; commit() writes them once the caller has
// issued its weight loads.
template <int XT> struct TStager {
  u32x4 d[4];
  int total, words, C;
  __device__ inline TStager(int nr, int K) : total(nr * (K >> 3)), words(K >> 3), C(K >> 5) {}
  template <class RowOf> __device__ inline void issue(RowOf row_of, int i0) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int idx = min(i0 + u * (int)blockDim.x + (int)threadIdx.x, total - 1);
      const int r = idx / words, m = idx - r * words;
      d[u] = ldg16(row_of(r) + 8 * m);
    }
  }
  __device__ inline void commit(int i0, u32x4* xs, float2* sums) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int idx = i0 + u * (int)blockDim.x + (int)threadIdx.x;
      if (idx < total) {
        const int r = idx / words, m = idx - r * words;
        const int o = (4 * r + (m & 3)) * C + (m >> 2);
        xs[o] = d[u];
        sums[o] = sum8n<XT>(d[u]);
      }
    }
  }
  template <class RowOf> __device__ inline void rest(RowOf row_of, u32x4* xs, float2* sums) {
    for (int i0 = 4 * (int)blockDim.x; i0 < total; i0 += 4 * (int)blockDim.x) {
      issue(row_of, i0);
      commit(i0, xs, sums);
    }
  }
};

// One lane's contribution of superchunk s against staged row x (word j of
// each chunk): sum over its 32 columns of (q - z) s x, corrected per group.
template <int XT, int ST, bool GB>
__device__ inline float tile_dot(const TSlot<GB>& sl, const u32x4* xs, const float2* sums,
                                 int s, int gshift, u32 mg) {
  float acc = 0.f, lo = 0.f, hi = 0.f, sb = 0.f, sp = 0.f;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const u32x4 xw = xs[4 * s + t];
    const float2 sm = sums[4 * s + t];
    dot8<XT>(word_t(sl.w, t), xw, lo, hi, mg);
    if constexpr (GB) {
      sb += sm.x;
      sp += sm.y;
    } else {
      const int g = (4 * s + t) >> gshift;
      const float a = fmaf(hi, hi_scale<XT>(), lo);
      acc = fmaf(scale_from_raw<ST>(sl.s[t]), a - Half<XT>::MAGIC * sm.x - zero_of(sl.z, g) * sm.y,
                 acc);
      lo = hi = 0.f;
    }
  }
  if constexpr (GB) {
    const int g = (4 * s) >> gshift;
    const float a = fmaf(hi, hi_scale<XT>(), lo);
    acc = scale_from_raw<ST>(sl.s[0]) * (a - Half<XT>::MAGIC * sb - zero_of(sl.z, g) * sp);
  }
  return acc;
}

// sum over the four k-groups of a row (lanes r, r + 16, r + 32, r + 48); every
// lane ends with its row's total
__device__ inline float kgroup_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
  const int src = ((int)__lane_id() ^ 32) << 2;
  return v + __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src, __builtin_bit_cast(int, v)));
}

}  // namespace i4
