// Device helpers shared by every gfx950 kernel of libi4moe.
//
// Nibble decode.  A CT word holds columns k0..k0+7 in nibbles 0..7.  The
// expression (w >> 4p) & 0x000F000F moves nibble p to bits 0..3 and nibble
// p+4 to bits 16..19; OR-ing the exponent pattern of a half-precision M turns
// the two 16-bit lanes into the exact values M + q (M = 1024 for fp16, whose
// ulp there is 1; M = 128 for bf16, whose ulp there is 1 as well).  One
// v_and_or_b32 (plus a shift) therefore yields a (k0+p, k0+p+4) pair ready
// for v_dot2_f32_{f16,bf16}, which multiplies exactly and accumulates in fp32.
// fp16 saves two shifts per word: w & 0x00F000F0 reads nibbles 1 and 5 in
// place as the exact values M + 16q (< 2048); those pairs accumulate
// separately and enter the chunk sum divided by 16.
// The bias M and the zero point z are removed per 32-column chunk with the
// chunk's activation sums: with S the plain sum and Sb the bias coefficient
// (S for bf16; S_lo + S_hi / 16 for fp16, lo = pairs 0 and 2),
//     sum (q - z) x = (lo + hi / 16) - M Sb - z S.
// Activations are staged once per workgroup in LDS, already permuted into the
// (k0+p, k0+p+4) pair order, together with (Sb, S) per chunk.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "i4moe.h"

namespace i4 {

typedef unsigned int u32;
typedef u32 u32x2 __attribute__((ext_vector_type(2)));
typedef u32 u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// 16-byte global load (global_load_dwordx4) of a packed-weight stream
__device__ inline u32x4 ldg16(const void* p) { return *(const u32x4*)p; }

// Raw buffer descriptors: base, size in bytes (loads past it return 0) and
// word 3 of a gfx9 descriptor for raw (untyped) dword access.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
static constexpr int kRawBuffer = 0x00020000;
__device__ inline rsrc_t rsrc(const void* base, u32 bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           kRawBuffer);
}

// Device-coherent accesses, for data that one workgroup of a launch hands to
// another: the two may run on different XCDs, each with its own L2, so the
// store writes through (sc1) and the load is served from memory, not from a
// line its own L2 may still hold (sc1).  No fence is involved: a consumer
// recognises finished data by its value (see the sentinel below).
static constexpr int kCoherent = 16;  // cache-policy bit sc1 of a buffer access
// A store with sc0 instead stays in its XCD's L2 (and reaches memory later), where a
// sc1 load from a CU of the same XCD finds it sooner than one written through.
static constexpr int kL2Only = 1;
__device__ inline u32x4 ld16_coherent(rsrc_t r, u32 voff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, kCoherent);
}
__device__ inline void st_coherent(uint16_t* p, uint16_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 0xFFFF is a NaN in fp16 and bf16 alike; producers that hand over halves
// this way write every NaN in its canonical form, so the pattern never
// occurs in finished data and marks a value not yet written.
static constexpr u32 kPending16 = 0xFFFFu;
__device__ inline bool has_pending(u32x4 d) {
  const u32 w[4] = {d.x, d.y, d.z, d.w};
  bool p = false;
#pragma unroll
  for (int i = 0; i < 4; ++i) p |= (w[i] & 0xFFFFu) == kPending16 || (w[i] >> 16) == kPending16;
  return p;
}

// The nibble decode computes (w & mask) | magic.  A gfx9 VOP3 instruction
// reads at most one SGPR and takes no literal, so with both operands constant
// the compiler emits v_and_b32 + v_or_b32; with the magic in a VGPR it is one
// v_and_or_b32.  magic_v() puts it there once, at kernel entry, in a way the
// optimizer cannot fold back into a constant; the decode itself stays plain
// code, so the compiler tracks every hazard around it.
__device__ inline u32 vgpr_const(u32 c) {
  u32 r;
  asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "s"(c));
  return r;
}

// ---------------------------------------------------------------------------
// half-precision codecs, selected by the I4_F16 / I4_BF16 dtype code
template <int DT> struct Half;

template <> struct Half<I4_F16> {
  static constexpr u32 MAGIC2 = 0x64006400u;  // two fp16 1024.0
  static constexpr uint16_t QNAN = 0x7E00u;   // canonical quiet NaN
  static constexpr float MAGIC = 1024.0f;
  __device__ static inline float to_f32(uint16_t b) {
    return (float)__builtin_bit_cast(_Float16, b);
  }
  __device__ static inline uint16_t from_f32(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
  }
  __device__ static inline float dot2(u32 a, u32 b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a),
                                  __builtin_bit_cast(f16x2, b), c, false);
  }
};

template <> struct Half<I4_BF16> {
  static constexpr u32 MAGIC2 = 0x43004300u;  // two bf16 128.0
  static constexpr uint16_t QNAN = 0x7FC0u;   // canonical quiet NaN
  static constexpr float MAGIC = 128.0f;
  __device__ static inline float to_f32(uint16_t b) {
    return __builtin_bit_cast(float, (u32)b << 16);
  }
  __device__ static inline uint16_t from_f32(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
  }
  __device__ static inline float dot2(u32 a, u32 b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                           __builtin_bit_cast(bf16x2, b), c, false);
  }
};

// scale element of any supported dtype, widened to fp32
template <int ST> __device__ inline float load_scale(const void* p, int64_t i) {
  if constexpr (ST == I4_F32) {
    return ((const float*)p)[i];
  } else {
    return Half<ST>::to_f32(((const uint16_t*)p)[i]);
  }
}

// Raw scale bits, loaded now and widened later so that a load never has to
// be waited for before the next one is issued.
template <int ST> __device__ inline u32 load_scale_raw(const void* p, int64_t i) {
  if constexpr (ST == I4_F32) return ((const u32*)p)[i];
  else return (u32)((const uint16_t*)p)[i];
}
template <int ST> __device__ inline float scale_from_raw(u32 r) {
  if constexpr (ST == I4_F32) return __builtin_bit_cast(float, r);
  else return Half<ST>::to_f32((uint16_t)r);
}

// Zero-point words of a symmetric weight (every nibble 8).  Kernels read
// zeros through a pointer that is either the caller's zeros or this table
// with zero strides, so the zero load is branch-free.  64 words cover
// K <= 16384 at group 32.  Kept non-const so it lives in the global address
// space and a select between it and a kernel argument stays a global load.
static __device__ u32 kSymZeros[64] = {
    0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u,
    0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u,
    0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u,
    0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u,
    0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u,
    0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u,
    0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u,
    0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u,
    0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u,
    0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u,
    0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};

// One 32-column chunk of one CT row: 4 packed words, its group's raw scale
// and the zero word holding its group's zero point.
struct Chunk {
  u32x4 w;
  u32 s, z;
};

// CT row view: packed row, scale row, zero row (already offset to the row)
struct RowPtr {
  const int32_t* p;
  const void* s;
  const u32* z;
};

template <int ST> __device__ inline const void* scale_at(const void* p, int64_t i) {
  return (const char*)p + i * (ST == I4_F32 ? 4 : 2);
}

template <int ST>
__device__ inline Chunk load_chunk(const RowPtr& r, int c, int gshift) {
  Chunk k;
  const int g = c >> gshift;
  k.w = *(const u32x4*)(r.p + 4 * c);
  k.s = load_scale_raw<ST>(r.s, g);
  k.z = r.z[g >> 3];
  return k;
}

// store one fp32 result in the requested output dtype
template <int OT> __device__ inline void store_out(void* p, int64_t i, float v) {
  if constexpr (OT == I4_F32) {
    ((float*)p)[i] = v;
  } else {
    ((uint16_t*)p)[i] = Half<OT>::from_f32(v);
  }
}

// ---------------------------------------------------------------------------
// nibble decode + dot of one CT word (8 columns) against its 4 staged x pairs;
// lo / hi accumulate the pairs as described at the top of this file.
template <int XT> __device__ inline void dot8(u32 w, u32x4 xp, float& lo, float& hi, u32 mg) {
  constexpr u32 MK = 0x000F000Fu;
  if constexpr (XT == I4_F16) {
    const u32 t = w >> 8;
    lo = Half<XT>::dot2((w & MK) | mg, xp.x, lo);
    hi = Half<XT>::dot2((w & 0x00F000F0u) | mg, xp.y, hi);
    lo = Half<XT>::dot2((t & MK) | mg, xp.z, lo);
    hi = Half<XT>::dot2((t & 0x00F000F0u) | mg, xp.w, hi);
  } else {
    lo = Half<XT>::dot2((w & MK) | mg, xp.x, lo);
    hi = Half<XT>::dot2(((w >> 4) & MK) | mg, xp.y, hi);
    lo = Half<XT>::dot2(((w >> 8) & MK) | mg, xp.z, lo);
    hi = Half<XT>::dot2(((w >> 12) & MK) | mg, xp.w, hi);
  }
}

// the decode magic of activation dtype XT in a VGPR (see vgpr_const)
template <int XT> __device__ inline u32 magic_v() { return vgpr_const(Half<XT>::MAGIC2); }

// hi-pair weight of the fp16 decode (its pairs carry 16q)
template <int XT> constexpr float hi_scale() { return XT == I4_F16 ? 1.0f / 16.0f : 1.0f; }

// the end of a chunk's dot: scale and zero applied to the decoded pair sums lo / hi
template <int XT, int ST>
__device__ inline float chunk_tail(float lo, float hi, u32 s, u32 zw, float2 sums, int c,
                                   int gshift) {
  const int g = c >> gshift;
  const float z = (float)((zw >> (4 * (g & 7))) & 15u);
  const float a = fmaf(hi, hi_scale<XT>(), lo);
  return scale_from_raw<ST>(s) * (a - Half<XT>::MAGIC * sums.x - z * sums.y);
}

// sum over one chunk of (q - z) * s * x given the chunk's staged x words
// (xw0..xw3, pair order) and its sums (Sb, S)
template <int XT, int ST>
__device__ inline float chunk_dot(const Chunk& k, u32x4 xw0, u32x4 xw1, u32x4 xw2, u32x4 xw3,
                                  float2 sums, int c, int gshift, u32 mg) {
  float lo = 0.f, hi = 0.f;
  dot8<XT>(k.w.x, xw0, lo, hi, mg);
  dot8<XT>(k.w.y, xw1, lo, hi, mg);
  dot8<XT>(k.w.z, xw2, lo, hi, mg);
  dot8<XT>(k.w.w, xw3, lo, hi, mg);
  return chunk_tail<XT, ST>(lo, hi, k.s, k.z, sums, c, gshift);
}

// A chunk with its nibbles already spread into the (nibble | magic) pairs that dot8
// builds, four per word in dot8's order: for a projection whose weights land before its
// activations, so the spreading runs while the activations are in flight.  xchunk_dot
// then does chunk_dot's products in chunk_dot's order (the same result bit for bit).
struct XChunk {
  u32 p[16];
  u32 s, z;
};

template <int XT> __device__ inline XChunk expand_chunk(const Chunk& k, u32 mg) {
  constexpr u32 MK = 0x000F000Fu;
  XChunk x;
  const u32 w4[4] = {k.w.x, k.w.y, k.w.z, k.w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u32 w = w4[i];
    if constexpr (XT == I4_F16) {
      const u32 t = w >> 8;
      x.p[4 * i] = (w & MK) | mg;
      x.p[4 * i + 1] = (w & 0x00F000F0u) | mg;
      x.p[4 * i + 2] = (t & MK) | mg;
      x.p[4 * i + 3] = (t & 0x00F000F0u) | mg;
    } else {
      x.p[4 * i] = (w & MK) | mg;
      x.p[4 * i + 1] = ((w >> 4) & MK) | mg;
      x.p[4 * i + 2] = ((w >> 8) & MK) | mg;
      x.p[4 * i + 3] = ((w >> 12) & MK) | mg;
    }
  }
  x.s = k.s;
  x.z = k.z;
  return x;
}

// keeps the spread pairs where they are computed: the compiler would otherwise move the
// spreading next to its use, past the wait it is meant to overlap
__device__ inline void pin(XChunk& x) {
#pragma unroll
  for (int i = 0; i < 16; ++i) asm volatile("" : "+v"(x.p[i]));
}

template <int XT, int ST>
__device__ inline float xchunk_dot(const XChunk& k, u32x4 xw0, u32x4 xw1, u32x4 xw2, u32x4 xw3,
                                   float2 sums, int c, int gshift) {
  float lo = 0.f, hi = 0.f;
  const u32x4 xw[4] = {xw0, xw1, xw2, xw3};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    lo = Half<XT>::dot2(k.p[4 * i], xw[i].x, lo);
    hi = Half<XT>::dot2(k.p[4 * i + 1], xw[i].y, hi);
    lo = Half<XT>::dot2(k.p[4 * i + 2], xw[i].z, lo);
    hi = Half<XT>::dot2(k.p[4 * i + 3], xw[i].w, hi);
  }
  return chunk_tail<XT, ST>(lo, hi, k.s, k.z, sums, c, gshift);
}

// Permute 8 consecutive half-precision x values (one 16-byte load, dwords
// d = (x0,x1),(x2,x3),(x4,x5),(x6,x7)) into the decode pair order
// (x0,x4),(x1,x5),(x2,x6),(x3,x7).  v_perm_b32 picks bytes of {src0:src1}.
__device__ inline u32x4 pair_order(u32x4 d) {
  u32x4 r;
  r.x = __builtin_amdgcn_perm(d.z, d.x, 0x05040100u);
  r.y = __builtin_amdgcn_perm(d.z, d.x, 0x07060302u);
  r.z = __builtin_amdgcn_perm(d.w, d.y, 0x05040100u);
  r.w = __builtin_amdgcn_perm(d.w, d.y, 0x07060302u);
  return r;
}

// (Sb, S) contribution of the 8 half values of one 16-byte load (see top)
template <int XT> __device__ inline float2 sum8(u32x4 d) {
  const float x0 = Half<XT>::to_f32((uint16_t)(d.x & 0xFFFF)), x1 = Half<XT>::to_f32((uint16_t)(d.x >> 16));
  const float x2 = Half<XT>::to_f32((uint16_t)(d.y & 0xFFFF)), x3 = Half<XT>::to_f32((uint16_t)(d.y >> 16));
  const float x4 = Half<XT>::to_f32((uint16_t)(d.z & 0xFFFF)), x5 = Half<XT>::to_f32((uint16_t)(d.z >> 16));
  const float x6 = Half<XT>::to_f32((uint16_t)(d.w & 0xFFFF)), x7 = Half<XT>::to_f32((uint16_t)(d.w >> 16));
  const float slo = ((x0 + x4) + (x2 + x6)), shi = ((x1 + x5) + (x3 + x7));
  return make_float2(fmaf(shi, hi_scale<XT>(), slo), slo + shi);
}

// (Sb, S) of 8 consecutive half values in their natural order, for words whose
// nibbles are interleaved (I4_LAYOUT_TILE): decode pair p then covers x
// dword p, so the "lo" pairs are dwords 0 and 2, the "hi" pairs dwords 1 and 3
template <int XT> __device__ inline float2 sum8n(u32x4 d) {
  const float x0 = Half<XT>::to_f32((uint16_t)(d.x & 0xFFFF)), x1 = Half<XT>::to_f32((uint16_t)(d.x >> 16));
  const float x2 = Half<XT>::to_f32((uint16_t)(d.y & 0xFFFF)), x3 = Half<XT>::to_f32((uint16_t)(d.y >> 16));
  const float x4 = Half<XT>::to_f32((uint16_t)(d.z & 0xFFFF)), x5 = Half<XT>::to_f32((uint16_t)(d.z >> 16));
  const float x6 = Half<XT>::to_f32((uint16_t)(d.w & 0xFFFF)), x7 = Half<XT>::to_f32((uint16_t)(d.w >> 16));
  const float slo = ((x0 + x1) + (x4 + x5)), shi = ((x2 + x3) + (x6 + x7));
  return make_float2(fmaf(shi, hi_scale<XT>(), slo), slo + shi);
}

// ---------------------------------------------------------------------------
// cross-lane sums over aligned groups of L lanes (L a power of two <= 64);
// every lane of the group ends with the group total.
template <int CTRL> __device__ inline float dpp_mov(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

template <int L> __device__ inline float group_sum(float v) {
  if constexpr (L >= 2) v += dpp_mov<0xB1>(v);    // quad_perm [1,0,3,2]
  if constexpr (L >= 4) v += dpp_mov<0x4E>(v);    // quad_perm [2,3,0,1]
  if constexpr (L >= 8) v += dpp_mov<0x141>(v);   // row_half_mirror
  if constexpr (L >= 16) v += dpp_mov<0x140>(v);  // row_mirror
  if constexpr (L >= 32)
    v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v),
                                                                0x401F));  // xor 16
  if constexpr (L >= 64) {
    const int src = ((int)__lane_id() ^ 32) << 2;
    v += __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src, __builtin_bit_cast(int, v)));
  }
  return v;
}

// Two-phase staging of nr activation rows (row r starts at row_of(r), K
// halves each) into LDS in decode pair order with per-chunk sums:
//   xs  [nr][4][C] uint4 (word jw of chunk c of row r at (r*4 + jw)*C + c),
//   sums[nr][C] float2 (Sb, S).
// issue() puts up to 4 loads per thread in flight and returns; the caller
// issues its weight loads next and only then commit()s, so the LDS writes
// wait for the activations alone (loads retire in issue order).
// NT: the workgroup size, a compile-time constant in the index arithmetic
// (every user launches 256 threads)
template <int XT, int NT = 256> struct Stager {
  u32x4 d[4];
  int total, words, C;
  __device__ inline Stager(int nr, int K) : total(nr * (K >> 3)), words(K >> 3), C(K >> 5) {}
  template <class RowOf> __device__ inline void issue(RowOf row_of, int i0) {
    constexpr int nt = NT;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int idx = min(i0 + u * nt + (int)threadIdx.x, total - 1);
      const int r = idx / words, m = idx - r * words;
      d[u] = ldg16(row_of(r) + 8 * m);
    }
  }
  __device__ inline void commit(int i0, u32x4* xs, float2* sums) {
    constexpr int nt = NT;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int idx = i0 + u * nt + (int)threadIdx.x;
      if (idx < total) {  // total and nt are multiples of 4: quads are all in or all out
        const int r = idx / words, m = idx - r * words;
        const int c = m >> 2, jw = m & 3;
        xs[(r * 4 + jw) * C + c] = pair_order(d[u]);
        float2 sm = sum8<XT>(d[u]);
        sm.x = group_sum<4>(sm.x);
        sm.y = group_sum<4>(sm.y);
        if (jw == 0) sums[r * C + c] = sm;
      }
    }
  }
  // everything beyond the first round (rows longer than 4 * NT words)
  template <class RowOf> __device__ inline void rest(RowOf row_of, u32x4* xs, float2* sums) {
    for (int i0 = 4 * NT; i0 < total; i0 += 4 * NT) {
      issue(row_of, i0);
      commit(i0, xs, sums);
    }
  }
};

// Polls for the activations of a handoff launch (one staging round: at most
// 4 x 256 16-byte words): the rows are loaded device-coherently until no value
// still holds the pending pattern (an earlier launch fills them with it;
// producer workgroups of the same launch overwrite every value).  Returns true
// if max_polls polls went by without that, which a launch whose workgroups are
// dispatched in block order never sees: the bound guarantees that every wave
// exits.  The barrier in each pass also keeps the loads inside the loop.
template <int XT>
__device__ inline bool poll_rows(Stager<XT, 256>& st, const uint16_t* src, int max_polls) {
  constexpr int nt = 256;
  const rsrc_t r = rsrc(src, (u32)st.total * 16u);
  for (int it = 0;; ++it) {
    bool pend = false;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int idx = min(u * nt + (int)threadIdx.x, st.total - 1);
      st.d[u] = ld16_coherent(r, (u32)idx * 16u);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) pend |= has_pending(st.d[u]);
    if (!__syncthreads_or(pend)) return false;
    if (it >= max_polls) return true;
    __builtin_amdgcn_s_sleep(1);
  }
}

// RMSNorm of 8 values (one 16-byte load): round(round(x * r) * w), the order
// of transformers' Qwen3OmniMoeThinkerTextRMSNorm.forward
// (modeling_qwen3_omni_moe.py:1388-1393 in transformers 5.15).
// x * r is rounded to fp32 before the conversion: the empty asm keeps the compiler
// from fusing the product into the conversion (v_fma_mixlo, one rounding), which it
// does in some instantiations and not in others, so that every kernel normalises
// alike and as torch does (an fp32 product, then .to(dtype)).
template <int XT> __device__ inline u32 norm_pair(u32 xp, u32 wp, float r) {
  float pa = Half<XT>::to_f32((uint16_t)xp) * r, pb = Half<XT>::to_f32((uint16_t)(xp >> 16)) * r;
  asm volatile("" : "+v"(pa), "+v"(pb));
  const float a = Half<XT>::to_f32(Half<XT>::from_f32(pa));
  const float b = Half<XT>::to_f32(Half<XT>::from_f32(pb));
  const u32 lo = Half<XT>::from_f32(a * Half<XT>::to_f32((uint16_t)wp));
  const u32 hi = Half<XT>::from_f32(b * Half<XT>::to_f32((uint16_t)(wp >> 16)));
  return lo | (hi << 16);
}

template <int XT> __device__ inline float sumsq8(u32x4 d) {
  float s = 0.f;
  const u32 w[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a = Half<XT>::to_f32((uint16_t)w[i]), b = Half<XT>::to_f32((uint16_t)(w[i] >> 16));
    s += a * a;
    s += b * b;
  }
  return s;
}

__device__ inline float silu(float g) { return g / (1.0f + expf(-g)); }


}  // namespace i4
