// Device pieces shared by the stack's slot kernel and the per-linear kernel:
// raw buffer resources, the per-lane registers of one unit and the decode +
// MFMA step of one unit (see tp_tiled_common.h for the device layout).
#pragma once
#include "tp_tiled_common.h"

namespace tp {

constexpr int kBufferFlags = 0x00020000;  // raw buffer, 32-bit data format
constexpr uint32_t kOutOfRange = 0x80000000u;
// Cache policy of the weight streams (path / member words, MW member words
// per lane and unit), which a launch reads exactly once.  At 2-3 bits per
// weight: sc0 | nt, streaming loads that leave the caches to the data every
// wave re-reads (z, row scales, descriptors); on the Qwen3-4B decode-step
// stack 256.4 us per GEMV launch against 263.5 us with the default policy
// (k=3), 239.2 against 244.2 us (k=2).  At 4 bits (MW = 6), where the
// stack is HBM-bound, the default policy: 332.5 us against 338.0 us.
constexpr int weight_policy(int MW) { return MW <= 4 ? 3 : 0; }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, kBufferFlags);
}

// fp16 entries row0 .. row0+3 of a per-row vector of n entries (row scales,
// bias) as two dwords, zero past n and zero when !ok.  A buffer load is
// range-checked per dword: the one 8-byte load returns zero for a dword that
// runs past the vector's end, which for odd n holds row n - 1 (with row n);
// that row is loaded again on its own (2 bytes, inside the range).
__device__ __forceinline__ u32x2_t load_rows4(__amdgpu_buffer_rsrc_t r, int row0, int n, bool ok) {
  u32x2_t w = __builtin_amdgcn_raw_buffer_load_b64(r, ok ? (uint32_t)row0 * 2u : kOutOfRange, 0, 0);
  const int last = n - 1;
  if (ok && (n & 1) && last >= row0 && last < row0 + 4) {  // (row0 is a multiple of 4: last - row0 is 0 or 2)
    const uint32_t h = __builtin_amdgcn_raw_buffer_load_b16(r, (uint32_t)last * 2u, 0, 0);
    if (last - row0 >= 2) w[1] = h;
    else w[0] = h;
  }
  return w;
}

template <int MW> struct MemberBuf;
template <> struct MemberBuf<2> {
  typedef u32x2_t type;
  static __device__ __forceinline__ type load(__amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t s) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, v, s, weight_policy(2));
  }
};
template <> struct MemberBuf<4> {
  typedef u32x4_t type;
  static __device__ __forceinline__ type load(__amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t s) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, v, s, weight_policy(4));
  }
};
// k=4: six words (the k=3 words, then one high-member word per path word)
struct MemberWords6 {
  u32x4_t lo;
  u32x2_t hi;
  __device__ __forceinline__ uint32_t operator[](int i) const { return i < 4 ? lo[i] : hi[i - 4]; }
};
template <> struct MemberBuf<6> {
  typedef MemberWords6 type;
  static __device__ __forceinline__ type load(__amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t s) {
    MemberWords6 m;
    m.lo = __builtin_amdgcn_raw_buffer_load_b128(r, v, s, weight_policy(6));
    m.hi = __builtin_amdgcn_raw_buffer_load_b64(r, v + 16u, s, weight_policy(6));
    return m;
  }
};

// Loads of one unit of one lane.
template <int MW, int NZ>
struct UnitRegs {
  u32x2_t X;
  typename MemberBuf<MW>::type M;
  u32x4_t Z[NZ];
};

// Column (inside a 64-column segment) of the first of the 8 K positions of
// MFMA i of a unit: word x = i / 4 holds columns 16x..16x+15 and
// 32+16x..32+16x+15; MFMA j = i % 4 takes 8 of them.
__host__ __device__ constexpr int mfma_col(int i) {
  return 16 * (i >> 2) + ((i & 2) ? 32 : 0) + ((i & 1) ? 8 : 0);
}

// One unit of one wave: decode 64 weights per lane, 8 MFMAs.  Word 1 is
// decoded first: its previous word is this lane's word 0, so the halo
// exchange needed by word 0 completes meanwhile.
template <int KB, int NS, int SB, int MW, int NZ>
__device__ __forceinline__ void slot_unit(const UnitRegs<MW, NZ>& g, const uint32_t provide, const int lane,
                                          const uint32_t laneoff, const uint32_t* table, float4_t* acc) {
  constexpr int SLOTS = 16 / SB;
  const uint32_t halo = (uint32_t)__shfl((int)provide, (lane + 48) & 63, 64);
  MemberWords<KB> m[2];
  split_members<KB>(g.M, m);
#pragma unroll
  for (int xi = 0; xi < 2; ++xi) {
    const int x = 1 - xi;
    u32x4_t A[4];
    if (x == 1) {
      decode_word<KB, NS>(g.X[1], g.X[0], m[1], table, laneoff, A);
    } else {
      const uint32_t P = ((halo >> 1) & 0x55555555u) | ((g.X[1] << 1) & 0xAAAAAAAAu);
      decode_word<KB, NS>(g.X[0], P, m[0], table, laneoff, A);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = 4 * x + j;
      const half8_t b = __builtin_bit_cast(half8_t, g.Z[i / SLOTS]);
      acc[i % SLOTS] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, A[j]), b,
                                                             acc[i % SLOTS], 0, 0, 0);
    }
  }
}

}  // namespace tp
