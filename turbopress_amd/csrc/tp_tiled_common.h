// Device code shared by the tiled decode-GEMV kernels (tp_tiled.hip: one to
// four linears per launch; tp_stack.hip: every linear of a decode step in one
// persistent launch).  See tp_tiled.hip for the device layout.
#pragma once

#include "tp_common.h"

#include <cstdlib>

namespace tp {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));

// Loads/stores through the global address space.  Pointers read from a
// device-side descriptor table are generic to the compiler; generic (flat)
// accesses count against both the vector-memory and the LDS wait counters,
// so an LDS wait would also drain every prefetch in flight.
#define TP_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ T gld(const T* p) {
  return *(const TP_GLOBAL T*)p;
}
template <typename T>
__device__ __forceinline__ void gst(T* p, T v) {
  *(TP_GLOBAL T*)p = v;
}
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint2 gld2(const void* p) {
  const u32x2_t v = *(const TP_GLOBAL u32x2_t*)p;
  return uint2{v.x, v.y};
}
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
// Loads of weight words, which a launch reads once (MW member words per lane
// and unit): streaming (non-temporal) at 2-3 bits per weight, which leaves
// the caches to the data that waves re-read; plain at 4 bits (MW = 6), where
// the decode-step stack is HBM-bound and streaming loads measured slower.
template <int MW>
__device__ __forceinline__ uint32_t gld_w(const uint32_t* p) {
  if constexpr (MW <= 4) return __builtin_nontemporal_load((const TP_GLOBAL uint32_t*)p);
  else return *(const TP_GLOBAL uint32_t*)p;
}
template <int MW>
__device__ __forceinline__ uint2 gld2_w(const uint32_t* p) {
  u32x2_t v;
  if constexpr (MW <= 4) v = __builtin_nontemporal_load((const TP_GLOBAL u32x2_t*)p);
  else v = *(const TP_GLOBAL u32x2_t*)p;
  return uint2{v.x, v.y};
}

constexpr int kTileRows = 16;
constexpr int kSegCols = 64;
constexpr int kWavesPerGroup = 8;                 // waves per workgroup
constexpr int kGroupThreads = 64 * kWavesPerGroup;
constexpr int kTableWords = 256 * 64;            // 64 KiB
constexpr int kMaxInlineLinears = 4;

__host__ __device__ constexpr int member_words(int bits) {
  return bits == 2 ? 2 : bits == 3 ? 4 : bits == 4 ? 6 : 0;
}

// v / c, correctly rounded, for the fp32 c = sqrt(hb) of a power-of-two
// block, from r = RN(1/c): q = RN(v r), then one correction step (Markstein:
// e = v - q c is exact, RN(q + e r) is the rounded quotient).  For v = +-0
// and +-inf the correction gives +0 and NaN, so q itself is the answer
// there.  Checked against IEEE division for every fp32 v and every
// c = fp32(sqrt(2^j)), j = 1..14: equal wherever |v / c| >= 2^-105 (below,
// the residual underflows, and both quotients round to the same fp16
// signed zero).
__device__ __forceinline__ float div_by_block_root(float v, float c, float r) {
  const float q = v * r;
  const float e = __builtin_fmaf(-q, c, v);
  const float q1 = __builtin_fmaf(e, r, q);
  return __builtin_amdgcn_classf(q, 0x264 /* -inf, -0, +0, +inf */) ? q : q1;
}

// The same quotient with the special cases settled by v_div_fixup_f32
// (one instruction instead of a class test and a select): the signed zero
// for v = +-0, the signed infinity for v = +-inf, otherwise the corrected
// quotient's magnitude with v's sign (its underflow clause needs
// exponent(v) - exponent(c) < -150, impossible for c <= 2^23).  It keeps v
// live to the end, which pushed one register-bound kernel into scratch; the
// stack rotation uses it.
__device__ __forceinline__ float div_by_block_root_fx(float v, float c, float r) {
  const float q = v * r;
  const float e = __builtin_fmaf(-q, c, v);
  const float q1 = __builtin_fmaf(e, r, q);
  return __builtin_amdgcn_div_fixupf(q1, c, v);
}

// Two fp32 values as two halves (low, high) of a word, each rounded to
// nearest like f2h: one v_cvt_pk_f16_f32.
__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
  typedef float f2_t __attribute__((ext_vector_type(2)));
  typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2_t{lo, hi}, h2_t));
}

// Lane xor 1, 2, 4 or 8 (inside a row of 16 lanes) with DPP moves: no LDS.
__device__ __forceinline__ float lane_xor_row(float v, int m) {
  const int x = __builtin_bit_cast(int, v);
  int y;
  if (m == 1) {
    y = __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
  } else if (m == 2) {
    y = __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
  } else if (m == 4) {
    // lanes 0-3 and 8-11 of a row read lane + 4 (row_shl:4), the others lane - 4 (row_shr:4)
    y = __builtin_amdgcn_mov_dpp(x, 0x104, 0xF, 0x5, false);
    y = __builtin_amdgcn_update_dpp(y, x, 0x114, 0xF, 0xA, false);
  } else {
    y = __builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, false);  // row_ror:8
  }
  return __builtin_bit_cast(float, y);
}

// a plus the b of lane l + W of the same row of 16 lanes (DPP row_ror:16-W).
template <int W>
__device__ __forceinline__ float add_rot(float a, float b) {
  static_assert(W >= 1 && W <= 8, "row rotation");
  const int y = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, b), 0x120 | (16 - W), 0xF, 0xF, true);
  return a + __builtin_bit_cast(float, y);
}
template <int N, int W>
__device__ __forceinline__ void slot_pair_levels(float4_t* t) {
  if constexpr (N > 1) {
#pragma unroll
    for (int j = 0; j < N / 2; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) t[j][i] = add_rot<W>(t[2 * j][i], t[2 * j + 1][i]);
    slot_pair_levels<N / 2, 2 * W>(t);
  }
}
// Column sums of the slot accumulators (SLOTS = 16 / SB, the lane of row
// position r holding its valid column in acc[r / SB]) for the lanes of slot
// 0: lane l (l % 16 < SB) gets acc[0] of lane l + acc[1] of lane l + SB +
// .. + acc[SLOTS-1] of lane l + (SLOTS-1) SB, added pairwise (adjacent
// slots, then adjacent pairs, ..).  Selecting acc[slot] in every lane and
// then adding lane v xor SB, 2 SB, .. (a butterfly) adds the same values in
// the same order, so for finite values the sums are bit-identical to that
// form, here with (SLOTS - 1) x 4 DPP adds and no selection.
template <int SLOTS, int SB>
__device__ __forceinline__ float4_t slot_column_sums(const float4_t* acc) {
  static_assert(SLOTS * SB == 16, "16 columns per row");
  float4_t t[SLOTS];
#pragma unroll
  for (int s = 0; s < SLOTS; ++s) t[s] = acc[s];
  slot_pair_levels<SLOTS, SB>(t);
  return t[0];
}

// One butterfly at lane distance 16 (K = 4) or 32 (K = 5) without LDS:
// v_permlane16_swap / v_permlane32_swap with both operands v leave the
// lower lane's value in r[0] and the upper lane's in r[1], in both lanes of
// each pair (16-lane rows 0-1 and 2-3 / the two 32-lane halves), so
// fma(sg, r[1], r[0]) is own + partner in the lower lane (sg = +1) and
// partner - own in the upper one (sg = -1): the same sum or difference of
// the same two values as fma(sg, own, partner) with a bpermute partner.
template <int K>
__device__ __forceinline__ float lane_swap_butterfly(float v, float sg) {
  static_assert(K == 4 || K == 5, "lane distance 16 or 32");
  const uint32_t x = __builtin_bit_cast(uint32_t, v);
  uint32_t lo, hi;
  if constexpr (K == 4) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    lo = r[0];
    hi = r[1];
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    lo = r[0];
    hi = r[1];
  }
  return __builtin_fmaf(sg, __builtin_bit_cast(float, hi), __builtin_bit_cast(float, lo));
}

// Delay mask of a window-coordinate generator: bit t set when the subset bit
// XORs in the path bit t columns back.
__host__ __device__ constexpr uint32_t delay_mask(uint32_t g, int m) {
  uint32_t gw = ((g >> m) & 1u) << m;
  for (int j = 0; j < m; ++j) gw |= ((g >> (m - 1 - j)) & 1u) << j;
  uint32_t dm = 0;
  for (int j = 0; j <= m; ++j)
    if ((gw >> j) & 1u) dm |= 1u << (m - j);
  return dm;
}

template <int NS> struct TrellisOf;
template <> struct TrellisOf<4> { static constexpr int m = 2; static constexpr uint32_t g0 = 05, g1 = 07; };
template <> struct TrellisOf<8> { static constexpr int m = 3; static constexpr uint32_t g0 = 015, g1 = 017; };
template <> struct TrellisOf<16> { static constexpr int m = 4; static constexpr uint32_t g0 = 023, g1 = 035; };
template <> struct TrellisOf<64> { static constexpr int m = 6; static constexpr uint32_t g0 = 0133, g1 = 0171; };

// Subset words of the two 16-weight groups carried by one interleaved path word.
// SA bit 2j / 2j+1 = subset bit 0 / 1 of first-half weight j; SB likewise for
// the second half.  `prev` is the interleaved word of the 16 preceding columns
// of each half.
template <int NS>
__device__ __forceinline__ void subset_words(uint32_t cur, uint32_t prev, uint32_t& SA, uint32_t& SB) {
  constexpr int m = TrellisOf<NS>::m;
  constexpr uint32_t D0 = delay_mask(TrellisOf<NS>::g0, m);
  constexpr uint32_t D1 = delay_mask(TrellisOf<NS>::g1, m);
  uint32_t sh[m + 1];
  sh[0] = cur;
#pragma unroll
  for (int t = 1; t <= m; ++t) sh[t] = __builtin_amdgcn_alignbit(cur, prev, 32 - 2 * t);
  uint32_t e0, e1;
  if constexpr (NS == 64) {
    // taps {0,1,2,4,5} and {0,1,4,5,6}: shared part first, three-input XORs
    static_assert(D0 == 0x37u && D1 == 0x73u, "S=64 generator taps");
    const uint32_t c = __builtin_amdgcn_bitop3_b32(sh[0], sh[1], sh[4], 0x96);
    e0 = __builtin_amdgcn_bitop3_b32(c, sh[5], sh[2], 0x96);
    e1 = __builtin_amdgcn_bitop3_b32(c, sh[5], sh[6], 0x96);
  } else {
    e0 = 0u;
    e1 = 0u;
#pragma unroll
    for (int t = 0; t <= m; ++t) {
      if ((D0 >> t) & 1u) e0 ^= sh[t];
      if ((D1 >> t) & 1u) e1 ^= sh[t];
    }
  }
  SA = (e0 & 0x55555555u) | ((e1 << 1) & 0xAAAAAAAAu);
  SB = ((e0 >> 1) & 0x55555555u) | (e1 & 0xAAAAAAAAu);
}

// LDS byte address of the lane's copy of table entry `byte b of idx` in
// table format f: (idx byte b) * 256 + byte f of laneoff.
template <int F = 0>
__device__ __forceinline__ uint32_t table_addr(uint32_t idx, uint32_t laneoff, int b) {
  return __builtin_amdgcn_perm(idx, laneoff, 0x0C0C0000u | ((4u + b) << 8) | (uint32_t)F);
}

// Lane offsets inside a 256-byte table row.  k=2: one format, 64 lane
// copies (byte 0 = lane * 4).  k=3: two formats of 32 copies each -- format
// 0 (subset nibble low, member nibble high) at bytes 0..127, format 1
// (member nibble low, subset nibble high) at 128..255 -- byte 0 / byte 1 of
// the returned word.
template <int KB>
__device__ __forceinline__ uint32_t lane_offsets(int lane) {
  if constexpr (KB == 4) {
    // 16 copies of 4 bytes per 64-byte row, the copy offset in every byte
    // (the high member bits of each pair are or-ed into bits 6..7)
    return ((uint32_t)(lane & 15) << 2) * 0x01010101u;
  } else if constexpr (KB == 3) {
    const uint32_t c = (uint32_t)(lane & 31) << 2;
    return c | ((128u + c) << 8);
  } else {
    return (uint32_t)lane << 2;
  }
}

// k=4: LDS byte address (idx byte b) * 256 + (byte b of the lane word).
__device__ __forceinline__ uint32_t table_addr4(uint32_t idx, uint32_t lanew, int b) {
  return __builtin_amdgcn_perm(idx, lanew, 0x0C0C0000u | ((4u + b) << 8) | (uint32_t)b);
}

__device__ __forceinline__ uint32_t lds_word(const uint32_t* table, uint32_t byte_addr) {
  return *reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(table) + byte_addr);
}

// Member words consumed with one interleaved path word (x = 0 or 1).
template <int KB> struct MemberWords;
template <> struct MemberWords<2> { uint32_t w; };
template <> struct MemberWords<3> { uint32_t a, b; };
template <> struct MemberWords<4> { uint32_t a, b, q; };

// Member words of interleaved path words x = 0, 1 from the member_words(KB)
// words of one segment.
template <int KB, typename W>
__device__ __forceinline__ void split_members(const W& w, MemberWords<KB> m[2]) {
  if constexpr (KB == 4) {
    m[0].a = w[0]; m[0].b = w[1]; m[1].a = w[2]; m[1].b = w[3]; m[0].q = w[4]; m[1].q = w[5];
  } else if constexpr (KB == 3) {
    m[0].a = w[0]; m[0].b = w[1]; m[1].a = w[2]; m[1].b = w[3];
  } else {
    m[0].w = w[0]; m[1].w = w[1];
  }
}

// Decode 32 weights (16 of each half) of one lane into four MFMA A operands:
// A[0]/A[1] = first-half columns 0-7 / 8-15, A[2]/A[3] = second half.
template <int KB, int NS>
__device__ __forceinline__ void decode_word(uint32_t cur, uint32_t prev, const MemberWords<KB>& M,
                                            const uint32_t* table, uint32_t laneoff, u32x4_t A[4]) {
  uint32_t SA, SB;
  subset_words<NS>(cur, prev, SA, SB);
  if constexpr (KB == 4) {
    // One table format: index byte [S0a S1a S0b S1b | M0a M1a M0b M1b] of the
    // low member bits (odd pairs shifted into place), the pair's two high
    // member bits into bits 6..7 of the lane-offset byte (row within the
    // index byte's 256-byte group).
    const uint32_t iae = (SA & 0x0F0F0F0Fu) | (M.a & 0xF0F0F0F0u);
    const uint32_t iao = ((SA >> 4) & 0x0F0F0F0Fu) | ((M.a << 4) & 0xF0F0F0F0u);
    const uint32_t ibe = (SB & 0x0F0F0F0Fu) | (M.b & 0xF0F0F0F0u);
    const uint32_t ibo = ((SB >> 4) & 0x0F0F0F0Fu) | ((M.b << 4) & 0xF0F0F0F0u);
    const uint32_t lae = (M.q & 0xC0C0C0C0u) | laneoff;
    const uint32_t lao = ((M.q << 2) & 0xC0C0C0C0u) | laneoff;
    const uint32_t lbe = ((M.q << 4) & 0xC0C0C0C0u) | laneoff;
    const uint32_t lbo = ((M.q << 6) & 0xC0C0C0C0u) | laneoff;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      A[0][2 * h] = lds_word(table, table_addr4(iae, lae, h));
      A[0][2 * h + 1] = lds_word(table, table_addr4(iao, lao, h));
      A[1][2 * h] = lds_word(table, table_addr4(iae, lae, 2 + h));
      A[1][2 * h + 1] = lds_word(table, table_addr4(iao, lao, 2 + h));
      A[2][2 * h] = lds_word(table, table_addr4(ibe, lbe, h));
      A[2][2 * h + 1] = lds_word(table, table_addr4(ibo, lbo, h));
      A[3][2 * h] = lds_word(table, table_addr4(ibe, lbe, 2 + h));
      A[3][2 * h + 1] = lds_word(table, table_addr4(ibo, lbo, 2 + h));
    }
  } else {
    uint32_t iae, iao, ibe, ibo;
    constexpr int FO = KB == 3 ? 1 : 0;  // table format of the odd-pair index words
    if constexpr (KB == 3) {
      // Member words are stored nibble-swapped within each byte, so one bit
      // select pairs every subset nibble with its member nibble: even pairs as
      // [subset | member << 4] (format 0), odd pairs as [member | subset << 4]
      // (format 1).
      iae = (SA & 0x0F0F0F0Fu) | (M.a & 0xF0F0F0F0u);
      iao = (SA & 0xF0F0F0F0u) | (M.a & 0x0F0F0F0Fu);
      ibe = (SB & 0x0F0F0F0Fu) | (M.b & 0xF0F0F0F0u);
      ibo = (SB & 0xF0F0F0F0u) | (M.b & 0x0F0F0F0Fu);
    } else {
      iae = (SA & 0x0F0F0F0Fu) | ((M.w << 4) & 0xF0F0F0F0u);
      iao = ((SA >> 4) & 0x0F0F0F0Fu) | (M.w & 0xF0F0F0F0u);
      ibe = (SB & 0x0F0F0F0Fu) | ((M.w << 2) & 0xF0F0F0F0u);
      ibo = ((SB >> 4) & 0x0F0F0F0Fu) | ((M.w >> 2) & 0xF0F0F0F0u);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      A[0][2 * h] = lds_word(table, table_addr<0>(iae, laneoff, h));
      A[0][2 * h + 1] = lds_word(table, table_addr<FO>(iao, laneoff, h));
      A[1][2 * h] = lds_word(table, table_addr<0>(iae, laneoff, 2 + h));
      A[1][2 * h + 1] = lds_word(table, table_addr<FO>(iao, laneoff, 2 + h));
      A[2][2 * h] = lds_word(table, table_addr<0>(ibe, laneoff, h));
      A[2][2 * h + 1] = lds_word(table, table_addr<FO>(ibo, laneoff, h));
      A[3][2 * h] = lds_word(table, table_addr<0>(ibe, laneoff, 2 + h));
      A[3][2 * h + 1] = lds_word(table, table_addr<FO>(ibo, laneoff, 2 + h));
    }
  }
}

// Pair table: 256 rows of 256 bytes; row v holds entry (cb[level_a] |
// cb[level_b] << 16) of index byte v in lane copies.  k=2: index byte v =
// [S0a S1a S0b S1b | Ma Mb ..], 64 copies.  k=3: format 0 (bytes 0..127, 32
// copies) reads v = [S0a S1a S0b S1b | M0a M1a M0b M1b], format 1 (bytes
// 128..255, 32 copies) the same fields with the nibbles swapped.
template <int KB>
__device__ __forceinline__ void pair_fields(uint32_t v, int fmt, uint32_t& sa, uint32_t& sb, uint32_t& ma,
                                            uint32_t& mb) {
  if constexpr (KB == 3) {
    const uint32_t s = fmt ? v >> 4 : v, m = fmt ? v : v >> 4;
    sa = s & 3u;
    sb = (s >> 2) & 3u;
    ma = m & 3u;
    mb = (m >> 2) & 3u;
  } else {
    (void)fmt;
    sa = v & 3u;
    sb = (v >> 2) & 3u;
    ma = (v >> 4) & 1u;
    mb = (v >> 5) & 1u;
  }
}

// k=4 table: 1024 rows of 64 bytes (16 lane copies); row 4v + m2a + 2 m2b
// holds (cb[level_a] | cb[level_b] << 16) for index byte v in format 0 and
// high member bits m2a, m2b (level = member * 4 + subset, member = low 2
// bits + 4 * high bit).  Run i (16 bytes) belongs to row i / 4.
__device__ __forceinline__ void pair_levels4(int i, uint32_t& la, uint32_t& lb) {
  const uint32_t row = (uint32_t)i >> 2, v = row >> 2;
  la = ((((v >> 4) & 3u) + 4u * (row & 1u)) << 2) | (v & 3u);
  lb = ((((v >> 6) & 3u) + 4u * ((row >> 1) & 1u)) << 2) | ((v >> 2) & 3u);
}

template <int KB>
__device__ void build_pair_table(uint32_t* table, const uint16_t* cb, int tid, int nthreads) {
  if constexpr (KB == 4) {
    for (int i = tid; i < kTableWords / 4; i += nthreads) {
      uint32_t la, lb;
      pair_levels4(i, la, lb);
      const uint32_t e = (uint32_t)cb[la] | ((uint32_t)cb[lb] << 16);
      u32x4_t run = {e, e, e, e};
      *reinterpret_cast<u32x4_t*>(table + 4 * i) = run;
    }
    return;
  }
  // Each thread writes 16-byte runs (4 lane copies) of one entry: 16 runs
  // per row, runs 8..15 are format 1 for k=3.
  for (int i = tid; i < kTableWords / 4; i += nthreads) {
    const uint32_t v = (uint32_t)(i >> 4);
    uint32_t sa, sb, ma, mb;
    pair_fields<KB>(v, (i & 15) >= 8, sa, sb, ma, mb);
    const uint32_t e = (uint32_t)cb[ma * 4 + sa] | ((uint32_t)cb[mb * 4 + sb] << 16);
    u32x4_t run = {e, e, e, e};
    *reinterpret_cast<u32x4_t*>(table + 4 * i) = run;
  }
}

// Reads through the constant address space: data a launch does not change,
// read at wave-uniform addresses, become scalar loads (a vector load would
// make every value derived from it per-lane, and its wait would also drain
// the weight loads in flight).
#define TP_CONST __attribute__((address_space(4)))

// This lane's codebook entry (cb[lane % 2^(KB+1)], the input of
// build_pair_table_lanes) through the scalar cache: the 2^(KB+1) fp16 entries
// are 2^KB dwords of a 4-byte aligned codebook, and the lane's entry is
// picked from scalar registers, so the table build waits for no vector load
// (the vector memory counter is in order: waiting for a load issued at the
// launch's start would also wait for every load issued after it).
template <int KB>
__device__ __forceinline__ uint32_t codebook_lane_scalar(const uint16_t* codebook, int lane) {
  constexpr int NW = 1 << KB;  // dwords of 2^(KB+1) fp16 entries
  const TP_CONST uint32_t* cbw = (const TP_CONST uint32_t*)codebook;
  uint32_t w[NW];
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    w[i] = cbw[i];
    // (kept a scalar value: else a select between two of them became a
    // per-lane vector load)
    __asm__ volatile("" : "+s"(w[i]));
  }
  const int e = lane & (2 * NW - 1);
  uint32_t v = w[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) v = (e >> 1) == i ? w[i] : v;
  return (e & 1) ? v >> 16 : v & 0xFFFFu;
}

// Same table from a codebook held one entry per lane (lane l has cb[l % 2^(KB+1)]):
// no memory reads, entries gathered with lane shuffles.
template <int KB>
__device__ void build_pair_table_lanes(uint32_t* table, uint32_t cb_lane, int tid, int nthreads) {
  if constexpr (KB == 4) {
    for (int i = tid; i < kTableWords / 4; i += nthreads) {
      uint32_t la, lb;
      pair_levels4(i, la, lb);
      const uint32_t lo = (uint32_t)__shfl((int)cb_lane, (int)la, 64);
      const uint32_t hi = (uint32_t)__shfl((int)cb_lane, (int)lb, 64);
      const uint32_t e = (lo & 0xFFFFu) | (hi << 16);
      u32x4_t run = {e, e, e, e};
      *reinterpret_cast<u32x4_t*>(table + 4 * i) = run;
    }
    return;
  }
  for (int i = tid; i < kTableWords / 4; i += nthreads) {
    const uint32_t v = (uint32_t)(i >> 4);
    uint32_t sa, sb, ma, mb;
    pair_fields<KB>(v, (i & 15) >= 8, sa, sb, ma, mb);
    const uint32_t lo = (uint32_t)__shfl((int)cb_lane, (int)(ma * 4 + sa), 64);
    const uint32_t hi = (uint32_t)__shfl((int)cb_lane, (int)(mb * 4 + sb), 64);
    const uint32_t e = (lo & 0xFFFFu) | (hi << 16);
    u32x4_t run = {e, e, e, e};
    *reinterpret_cast<u32x4_t*>(table + 4 * i) = run;
  }
}

struct MemberLoad2 { uint2 v; };
struct MemberLoad3 { uint4 v; };

// ---------------------------------------------------------------------------
// descriptors
// ---------------------------------------------------------------------------
constexpr int kChunkCols = 256;                   // columns per unit (4 segments)
constexpr int kMaxUnitsPerBlock = 2;              // K extent of one block <= 512 columns
constexpr int kZCols = kChunkCols * kMaxUnitsPerBlock;
constexpr int kTableBytes = kTableWords * 4;

struct LinearDesc {
  const uint32_t* path;    // [T][G][16][2]
  const uint32_t* member;  // [T][G][16][MW]
  const uint16_t* x;       // activations fp16 [batch][ldx]: unrotated (fused) or rotated z
  const uint16_t* rs;      // rot_scale fp16 [d] (fused rotation only)
  const uint16_t* scales;  // fp16 [n]
  const uint16_t* bias;    // fp16 [n] or null
  uint16_t* y;             // fp16 [batch][ldy]
  float* ws;               // [T*16][16*NBT] fp32 split-K sums (kept zero between calls)
  uint32_t* cnt;           // [T] split-K unit counters (kept zero between calls)
  uint16_t* z;             // stack plans: rotated activations fp16 [batch][G4 * 256]
  float hdiv;              // fp32(sqrt(hb))
  int32_t n, d, T, G, G4;
  int32_t ldx, ldy, kg, blocks;  // kg: units per block; blocks: ceil(T/8)*ceil(G4/kg)
  int32_t hb;              // Hadamard block
};


// z staging in LDS: [16*NBT rows][kZCols] halves, 16-byte chunks XOR-swizzled
// by row so that 16 batch rows reading the same column hit distinct banks.
__device__ __forceinline__ int zl_index(int row, int col) {
  return row * kZCols + ((((col >> 3) ^ (row & 15)) << 3) | (col & 7));
}

__device__ __forceinline__ void load4h(const uint16_t* p, float v[4]) {
  const uint2 w = gld2((p));
  v[0] = h2f((uint16_t)w.x);
  v[1] = h2f((uint16_t)(w.x >> 16));
  v[2] = h2f((uint16_t)w.y);
  v[3] = h2f((uint16_t)(w.y >> 16));
}

// One 256-column chunk of z = blockFWHT(x * rs) / sqrt(hb) for batch row b,
// computed by one wave (4 columns per lane, lane-major).  Columns >= d are
// zero.  For hb > 256 the chunk is row block o of H_hb = H_(hb/256) (x) H_256:
// first the signed sum of the hb/256 input chunks, then H_256.
__device__ void rotate_chunk(const LinearDesc& L, int b, int cs, int lane, float v[4]) {
  const int hb = L.hb;
  const uint16_t* xr = L.x + (size_t)b * L.ldx;
  v[0] = v[1] = v[2] = v[3] = 0.f;
  if (hb <= kChunkCols) {
    const int c0 = cs + lane * 4;
    if (c0 + 3 < L.d) {
      float xv[4], rv[4];
      load4h(xr + c0, xv);
      load4h(L.rs + c0, rv);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = xv[e] * rv[e];
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (c0 + e < L.d) v[e] = h2f(gld(xr + c0 + e)) * h2f(gld(L.rs + c0 + e));
    }
  } else {
    const int base = cs - cs % hb;
    const int o = (cs % hb) / kChunkCols;
    const int nsub = hb / kChunkCols;
    for (int i = 0; i < nsub; ++i) {
      const int c0 = base + i * kChunkCols + lane * 4;
      float xv[4], rv[4];
      load4h(xr + c0, xv);
      load4h(L.rs + c0, rv);
      const bool neg = __popc(i & o) & 1;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] += neg ? -(xv[e] * rv[e]) : xv[e] * rv[e];
    }
  }
  const int hmax = hb < kChunkCols ? hb : kChunkCols;
  if (hmax > 1) {
    float a = v[0], c = v[1];
    v[0] = a + c; v[1] = a - c;
    a = v[2]; c = v[3];
    v[2] = a + c; v[3] = a - c;
  }
  if (hmax > 2) {
    float a = v[0], c = v[2];
    v[0] = a + c; v[2] = a - c;
    a = v[1]; c = v[3];
    v[1] = a + c; v[3] = a - c;
  }
#pragma unroll
  for (int sft = 0; sft < 6; ++sft) {
    if ((4 << sft) >= hmax) break;
    const bool upper = (lane >> sft) & 1;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float p = __shfl_xor(v[e], 1 << sft, 64);
      v[e] = upper ? p - v[e] : v[e] + p;
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = v[e] / L.hdiv;
}

// Activations of one staging item loaded ahead of the block's LDS work: the
// common small case (at most one item per wave, Hadamard block <= 512) keeps
// every load of the block in flight before the first barrier.
struct ZPrefetch {
  bool valid;   // this wave stages an item of the chunk
  bool inb;     // the lane's 4 columns lie inside d (else they read as zero)
  uint2 x0, r0, x1, r1;
};

// Branch-free: every wave always issues its four loads from clamped, valid
// addresses (loads issued under divergent control flow would have to be
// waited for where their registers merge), and validity travels as flags.
template <bool ROT>
__device__ __forceinline__ ZPrefetch prefetch_z(const LinearDesc& L, int gu0, int ngu, int batch,
                                                int wave, int lane) {
  ZPrefetch zp;
  const int items = ngu * batch;
  zp.valid = !(items > kWavesPerGroup || wave >= items || (ROT && L.hb > 2 * kChunkCols));
  const int it = zp.valid ? wave : 0;
  const int ci = it / batch, b = it - ci * batch;
  const int cs = (gu0 + ci) * kChunkCols;
  if constexpr (ROT) {
    const uint16_t* xr = L.x + (size_t)b * L.ldx;
    const bool big = L.hb > kChunkCols;
    int c0 = (big ? cs - cs % L.hb : cs) + lane * 4;
    zp.inb = c0 < L.d;
    c0 = zp.inb ? c0 : 0;
    const int c1 = big ? c0 + kChunkCols : c0;
    zp.x0 = gld2(xr + c0);
    zp.r0 = gld2(L.rs + c0);
    zp.x1 = gld2(xr + c1);
    zp.r1 = gld2(L.rs + c1);
  } else {
    zp.inb = true;
    zp.x0 = gld2(L.x + (size_t)b * L.ldx + cs + lane * 4);
    zp.r0 = zp.x1 = zp.r1 = uint2{0u, 0u};
  }
  return zp;
}

__device__ __forceinline__ void unpack4h(uint2 w, float v[4]) {
  v[0] = h2f((uint16_t)w.x);
  v[1] = h2f((uint16_t)(w.x >> 16));
  v[2] = h2f((uint16_t)w.y);
  v[3] = h2f((uint16_t)(w.y >> 16));
}

// H_256 (or H_hb for hb < 256) butterflies over a lane-major chunk, then 1/sqrt(hb).
__device__ __forceinline__ void chunk_fwht(const LinearDesc& L, int lane, float v[4]) {
  const int hb = L.hb;
  const int hmax = hb < kChunkCols ? hb : kChunkCols;
  if (hmax > 1) {
    float a = v[0], c = v[1];
    v[0] = a + c; v[1] = a - c;
    a = v[2]; c = v[3];
    v[2] = a + c; v[3] = a - c;
  }
  if (hmax > 2) {
    float a = v[0], c = v[2];
    v[0] = a + c; v[2] = a - c;
    a = v[1]; c = v[3];
    v[1] = a + c; v[3] = a - c;
  }
#pragma unroll
  for (int sft = 0; sft < 6; ++sft) {
    if ((4 << sft) >= hmax) break;
    const bool upper = (lane >> sft) & 1;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float p = __shfl_xor(v[e], 1 << sft, 64);
      v[e] = upper ? p - v[e] : v[e] + p;
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = v[e] / L.hdiv;
}

template <bool ROT>
__device__ void stage_z_prefetched(const LinearDesc& L, int gu0, int batch, uint16_t* zl,
                                   int wave, int lane, const ZPrefetch& zp) {
  const int ci = wave / batch, b = wave - ci * batch;
  uint2 w;
  if constexpr (ROT) {
    float v[4], xv[4], rv[4];
    unpack4h(zp.x0, xv);
    unpack4h(zp.r0, rv);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = zp.inb ? xv[e] * rv[e] : 0.f;
    if (L.hb > kChunkCols) {  // hb == 512: row block o of H_2 (x) H_256
      const int o = (((gu0 + ci) * kChunkCols) % L.hb) / kChunkCols;
      unpack4h(zp.x1, xv);
      unpack4h(zp.r1, rv);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] += o ? -(xv[e] * rv[e]) : xv[e] * rv[e];
    }
    chunk_fwht(L, lane, v);
    w.x = (uint32_t)f2h(v[0]) | ((uint32_t)f2h(v[1]) << 16);
    w.y = (uint32_t)f2h(v[2]) | ((uint32_t)f2h(v[3]) << 16);
  } else {
    w = zp.x0;
  }
  *reinterpret_cast<uint2*>(zl + zl_index(b, ci * kChunkCols + lane * 4)) = w;
}

template <bool ROT>
__device__ void stage_z(const LinearDesc& L, int gu0, int ngu, int batch, uint16_t* zl,
                        int wave, int lane) {
  const int items = ngu * batch;
  for (int it = wave; it < items; it += kWavesPerGroup) {
    const int ci = it / batch;
    const int b = it - ci * batch;
    const int cs = (gu0 + ci) * kChunkCols;
    uint2 w;
    if constexpr (ROT) {
      float v[4];
      rotate_chunk(L, b, cs, lane, v);
      w.x = (uint32_t)f2h(v[0]) | ((uint32_t)f2h(v[1]) << 16);
      w.y = (uint32_t)f2h(v[2]) | ((uint32_t)f2h(v[3]) << 16);
    } else {
      w = gld2((L.x + (size_t)b * L.ldx + cs + lane * 4));
    }
    *reinterpret_cast<uint2*>(zl + zl_index(b, ci * kChunkCols + lane * 4)) = w;
  }
}

// One linear of a host-side launch (rotation fused when rot_scale is set).
struct TiledLinearArgs {
  const uint8_t* path_tiled;
  const uint8_t* member_tiled;
  const uint16_t* x;     // rotated z (rot_scale == null) or raw activations (fused rotation)
  int64_t ldx;
  const uint16_t* rot_scale;
  int64_t block;         // Hadamard block (fused rotation)
  const uint16_t* scales;
  const uint16_t* bias;
  uint16_t* y;
  int64_t ldy;
  int64_t n, d;
  void* workspace;
  int64_t workspace_bytes;
};

// Batch <= 8 decode-GEMV of 1..4 linears on one input in one pass
// (tp_linear.hip), for arguments the caller has validated.  Returns a status,
// or kLinearNotHandled when the shapes need the split-K kernel instead.
// With one linear, Hadamard blocks <= 512 columns and a workspace, the K
// range may also be cut into parts summed through the workspace (at most
// linear_ksplit_bytes(T) of it, left zero); clear_ws zeroes that region
// before the launch (for callers whose workspace may hold anything).
constexpr int kLinearNotHandled = 1 << 20;
int linear_forward_fast(const TiledLinearArgs* ls, int n_lin, int64_t batch, const uint16_t* codebook,
                        int bits, int n_states, hipStream_t s, bool clear_ws);
int64_t linear_ksplit_bytes(int64_t T);

// Zero `bytes` (a multiple of 4) of device memory with a fill kernel on
// stream s (a kernel node rather than a memset node under graph capture).
int zero_device_bytes(void* p, int64_t bytes, hipStream_t s);

// tp_packed_linear_forward on a workspace that may hold anything: every
// launch that uses it is preceded by a fill of the bytes it uses.
int packed_linear_forward_cleared(const uint16_t* x, int64_t ldx, int64_t batch, const uint16_t* rot_scale,
                                  int64_t block, const uint8_t* path_tiled, const uint8_t* member_tiled,
                                  const uint16_t* scales, const uint16_t* codebook, const uint16_t* bias, int64_t n,
                                  int64_t d, int bits, int n_states, uint16_t* y, int64_t ldy, void* workspace,
                                  int64_t workspace_bytes, void* stream);

// Batch 9..32 decode-GEMV of one linear, in 16-tile blocks, K split across
// workgroups through the workspace (tp_gemv_workspace_bytes) when one is
// given (tp_stack.hip): on rotated activations (z fp16 [batch][zld], zero
// past d), or with z null on L.x / L.rs, rotated in the launch (Hadamard
// block <= 512, d and ldx multiples of 8, 16-byte aligned x and rot_scale).
// Returns a status, or kLinearNotHandled for other batches or layouts.
int linear_forward_wide(const LinearDesc& L, const uint16_t* z, int64_t zld, int64_t batch,
                        const uint16_t* codebook, int bits, int n_states, void* workspace, int64_t workspace_bytes,
                        hipStream_t s);

// ---------------------------------------------------------------------------
// host-side geometry
// ---------------------------------------------------------------------------
struct Geom {
  int64_t T, G, G4, path_words, member_words;
};

inline int tiled_geom(int64_t n, int64_t d, int bits, Geom* g) {
  if (n <= 0 || d <= 0) return TP_ERR_BAD_DIMS;
  if (bits < 2 || bits > 4) return TP_ERR_UNSUPPORTED_BITS;
  g->T = (n + kTileRows - 1) / kTileRows;
  g->G4 = (d + 4 * kSegCols - 1) / (4 * kSegCols);
  g->G = 4 * g->G4;
  g->path_words = g->T * g->G * kTileRows * 2;
  g->member_words = g->T * g->G * kTileRows * member_words(bits);
  if (g->T > (1 << 26) || g->G > (1 << 20)) return TP_ERR_BAD_DIMS;
  return TP_OK;
}



// One unit (16 rows x 4 segments) of one wave: halo exchange, decode of the
// lane's 64 weights into MFMA A operands, B operands from the staged z (lc =
// column of this lane's segment inside the staged chunk), 8 MFMAs per batch
// tile into acc.
template <int KB, int NS, int NBT>
__device__ __forceinline__ void process_unit(const uint2 X, const uint32_t* Mw, const uint32_t x1_last,
                                             const int gu, const int lc, const int q, const int r,
                                             const int lane, const uint32_t laneoff,
                                             const uint32_t* table, const uint16_t* zl,
                                             const int batch, float4_t* acc) {
  // Halo: X1 of the previous segment, from the lane 16 below (K block q-1),
  // or for q == 0 from the last K block's previous unit; zero at a row start.
  const uint32_t provide = (q == 3) ? (gu == 0 ? 0u : x1_last) : X.y;
  const uint32_t halo = (uint32_t)__shfl((int)provide, (lane + 48) & 63, 64);
  const uint32_t P = ((halo >> 1) & 0x55555555u) | ((X.y << 1) & 0xAAAAAAAAu);
  MemberWords<KB> m[2];
  split_members<KB>(Mw, m);
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    // B operands of this interleaved word's 4 MFMAs (batch column r).
    half8_t zb[NBT][4];
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt) {
      const int nb = bt * 16 + r;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int off = 16 * x + (j & 2 ? 32 : 0) + (j & 1 ? 8 : 0);
        if (nb < batch)
          zb[bt][j] = *reinterpret_cast<const half8_t*>(zl + zl_index(nb, lc + off));
        else
          zb[bt][j] = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
      }
    }
    u32x4_t A[4];
    decode_word<KB, NS>(x ? X.y : X.x, x ? X.x : P, m[x], table, laneoff, A);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const half8_t av = __builtin_bit_cast(half8_t, A[j]);
#pragma unroll
      for (int bt = 0; bt < NBT; ++bt)
        acc[bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, zb[bt][j], acc[bt], 0, 0, 0);
    }
  }
}

}  // namespace tp
