// The transform of one 4096-column tile of rotated activations, z =
// blockFWHT(x * rot_scale) / sqrt(hb) for Hadamard blocks of at most 4096
// columns, shared by the stack's rotation launch (tp_stack.hip) and the
// per-linear launches that stage blocks of 1024..4096 columns (tp_linear.hip).
// 256 threads (4 waves) hold a tile; every butterfly is the reference's
// (distance 1, 2, 4, ... in order, a + b and a - b in fp32), so z is bit
// for bit the reference's transform.
//
// Thread (wave w, lane l) holds tile columns 1024 w + 256 g + 4 m(l) + j,
// g, j = 0..3: every 8-byte load or store of the wave covers 512
// contiguous bytes.  (Threads holding 16 contiguous columns measured the
// same; 32 or 64 contiguous columns per thread, fewer lane stages but 32 or
// 64 cache lines per load, took 37.6 / 48.3 us against 24 for the stack's
// batch-32 rotation.)  Butterflies at distance 1, 2 (j) and 256, 512 (g)
// run in registers, 4 .. 128 across lanes (bits of m), 1024 and 2048 as
// one radix-4 step through LDS (the wave).  m(l) puts lanes so that the
// partner of m bits 0..3 is one DPP move: lane xor 1 / 2 / 7 / 8 (two quad
// permutes, the half-row mirror, a row rotation by 8); bits 4 and 5 are
// lane xor 16 and 32 (a permlane swap or a bpermute each, see
// rot_lane_stage).  Stages are unrolled per block size
// (template LOGH = log2 hb), so that no stage is skipped at run time.
#pragma once
#include "tp_slot.h"

namespace tp {

constexpr int kRotTile = 4096;
constexpr int kRotThreads = 256;
constexpr int kRotEPT = kRotTile / kRotThreads;  // 16 columns per thread
constexpr int kRotMaxLogH = 12;                  // packed tiles: blocks of 1 .. 4096

// m(l): lane bits 0 and 1 xor lane bit 2 (so that m bit 2 is lane xor 7),
// every other bit as is.  The map is its own inverse.
__device__ __forceinline__ int rot_lane_index(int lane) { return lane ^ (((lane >> 2) & 1) * 3); }

// Tile column of element e (= 4 g + j) of thread (w, m).
__device__ __forceinline__ int rot_col(int w, int m, int e) { return 1024 * w + 256 * (e >> 2) + 4 * m + (e & 3); }

// The value of the lane whose m differs in bit K (K = 0..5); `lane4` is
// the lane index times 4 (the byte address of a bpermute).
template <int K>
__device__ __forceinline__ float rot_partner(float v, int lane4) {
  const int x = __builtin_bit_cast(int, v);
  int y;
  if constexpr (K == 0) y = __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false);        // quad_perm [1,0,3,2]
  else if constexpr (K == 1) y = __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
  else if constexpr (K == 2) y = __builtin_amdgcn_mov_dpp(x, 0x141, 0xF, 0xF, false);  // row_half_mirror
  else if constexpr (K == 3) y = __builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, false);  // row_ror:8
  else y = __builtin_amdgcn_ds_bpermute(lane4 ^ (4 << K), x);                         // lane xor 16 / 32
  return __builtin_bit_cast(float, y);
}

// Butterflies at distance 4 << K across lanes, when that is below the
// block: the lane whose m has bit K set keeps partner - own, the other
// own + partner, each one FMA fma(+-1, own, partner) (the product is exact,
// so the sum rounds as the add or subtract does).
//
// SWAP: distances 16 and 32 lanes by permlane swaps (VALU, no LDS: shorter
// latency, for launches that are one latency chain), else by bpermute (an
// LDS instruction beside one VALU FMA: for launches bound by VALU issue).
template <int K, int LOGH, int N = kRotEPT, bool SWAP = true>
__device__ __forceinline__ void rot_lane_stage(float* v, int m, int lane4) {
  if constexpr ((4 << K) < (1 << LOGH)) {
    // +-1.0: the sign bit from bit K of m
    const float sg = __builtin_bit_cast(float, 0x3F800000u | (((uint32_t)m << (31 - K)) & 0x80000000u));
#pragma unroll
    for (int e = 0; e < N; ++e) {
      if constexpr (K >= 4 && SWAP) v[e] = lane_swap_butterfly<K>(v[e], sg);  // (m bits 4, 5 are lane bits 4, 5)
      else v[e] = __builtin_fmaf(sg, v[e], rot_partner<K>(v[e], lane4));
    }
  }
}

// Butterflies between elements e and e + S (element stride S = 2: column
// distance 2; S = 4, 8: column distance 256, 512) when that distance is
// below the block.
template <int S, int DIST, int LOGH, int N = kRotEPT>
__device__ __forceinline__ void rot_reg_stage(float* v) {
  if constexpr (DIST < (1 << LOGH)) {
#pragma unroll
    for (int e = 0; e < N; ++e) {
      if ((e & S) == 0) {
        const float a = v[e], c = v[e + S];
        v[e] = a + c;
        v[e + S] = a - c;
      }
    }
  }
}

__device__ __forceinline__ float hlo(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)w); }
__device__ __forceinline__ float hhi(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
}

// v = x * rot_scale of G groups of 4 columns (4 halves each, as loaded; a
// thread of a 256-thread tile holds 4) with the distance-1 butterflies when
// the block has them: the
// product of two fp16 values is exact in fp32, so fma(x0, r0, +-x1 r1)
// rounds as the add / subtract of the two products does.
template <bool STAGE1, int G = kRotEPT / 4>
__device__ __forceinline__ void rot_products(const u32x2_t* xw, const u32x2_t* rw, float* v) {
  // x1 r1 as fma(x1, r1, -0) (exact; a -0 product keeps its sign), the -0 in
  // an opaque register: a literal one lets the compiler turn the fma into a
  // product of two converted halves (three instructions, not one)
  float nz = -0.f;
  __asm__("" : "+v"(nz));
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const uint32_t xv = xw[g][w], rv = rw[g][w];
      float* o = v + 4 * g + 2 * w;
      const float b = __builtin_fmaf(hhi(xv), hhi(rv), nz);
      if (STAGE1) {
        o[0] = __builtin_fmaf(hlo(xv), hlo(rv), b);
        o[1] = __builtin_fmaf(hlo(xv), hlo(rv), -b);
      } else {
        o[0] = __builtin_fmaf(hlo(xv), hlo(rv), nz);
        o[1] = b;
      }
    }
  }
}

// The stages of a block of 2^LOGH columns (at most 4096) from distance 2
// (rot_products ran the first) to 512, unnormalized: registers and lanes
// only.
template <int LOGH, bool SWAP = true>
__device__ __forceinline__ void rot_stages_lanes(float v[kRotEPT], int m, int lane4) {
  rot_reg_stage<2, 2, LOGH>(v);
  rot_lane_stage<0, LOGH, kRotEPT, SWAP>(v, m, lane4);
  rot_lane_stage<1, LOGH, kRotEPT, SWAP>(v, m, lane4);
  rot_lane_stage<2, LOGH, kRotEPT, SWAP>(v, m, lane4);
  rot_lane_stage<3, LOGH, kRotEPT, SWAP>(v, m, lane4);
  rot_lane_stage<4, LOGH, kRotEPT, SWAP>(v, m, lane4);
  rot_lane_stage<5, LOGH, kRotEPT, SWAP>(v, m, lane4);
  rot_reg_stage<4, 256, LOGH>(v);
  rot_reg_stage<8, 512, LOGH>(v);
}

// Distances 1024 (and 2048) of a block of 2^LOGH > 1024 columns: the bits
// of w (0..3, the wave inside the 4-wave tile group) through `ex` (4096
// floats of LDS per tile group) as one radix-4 step.  Every wave of the
// workgroup passes both barriers; only those with `act` read and write ex.
template <int LOGH>
__device__ __forceinline__ void rot_stage_waves(float v[kRotEPT], int w, int m, float* ex, bool act) {
  constexpr int HB = 1 << LOGH;
  static_assert(HB > 1024 && HB <= 4096, "the wave stages of a 2048- or 4096-column block");
  __syncthreads();  // the previous tile's reads of ex are done
  if (act) {
#pragma unroll
    for (int e = 0; e < kRotEPT; ++e) ex[rot_col(w, m, e)] = v[e];
  }
  __syncthreads();
  if (act) {
    const float s1 = (w & 1) ? -1.f : 1.f;
    if constexpr (HB == 2048) {
#pragma unroll
      for (int e = 0; e < kRotEPT; ++e) v[e] = __builtin_fmaf(s1, v[e], ex[rot_col(w ^ 1, m, e)]);
    } else {
      const float s2 = (w & 2) ? -1.f : 1.f;
#pragma unroll
      for (int e = 0; e < kRotEPT; ++e) {
        const int i0 = rot_col(0, m, e);
        const float u0 = ex[i0], u1 = ex[1024 + i0], u2 = ex[2048 + i0], u3 = ex[3072 + i0];
        // natural-order H_4 row w: stage 1024 then stage 2048
        const float s01 = __builtin_fmaf(s1, u1, u0);
        const float s23 = __builtin_fmaf(s1, u3, u2);
        v[e] = __builtin_fmaf(s2, s23, s01);
      }
    }
  }
}

// Every stage of a block of 2^LOGH columns (at most 4096) from distance 2,
// all 256 threads of the workgroup on one tile.
template <int LOGH, bool SWAP = true>
__device__ __forceinline__ void rot_stages(float v[kRotEPT], int w, int m, int lane4, float* ex) {
  rot_stages_lanes<LOGH, SWAP>(v, m, lane4);
  if constexpr ((1 << LOGH) > 1024) rot_stage_waves<LOGH>(v, w, m, ex, true);
}

// z of 4 columns of a block of 2^LOGH columns, v / sqrt(hb) correctly
// rounded (for even LOGH sqrt(hb) is a power of two and the product with
// its reciprocal is the quotient), as 4 halves.
template <int LOGH>
__device__ __forceinline__ u32x2_t rot_z4(const float* v, float c, float r) {
  float q[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) q[e] = (LOGH & 1) ? div_by_block_root_fx(v[e], c, r) : v[e] * r;
  return u32x2_t{pack_h2(q[0], q[1]), pack_h2(q[2], q[3])};
}

// Four halves (as two words) at element offset `o` of a buffer (out of
// range: zeros).
// Each load keeps its own opaque offset register so that the compiler does
// not merge two into one 16-byte access, which could straddle the end of
// the buffer (every d is a multiple of 4, so a group is wholly inside or
// outside).
__device__ __forceinline__ u32x2_t load4h_words(__amdgpu_buffer_rsrc_t r, uint32_t o) {
  uint32_t b = o * 2u;
  __asm__("" : "+v"(b));
  return __builtin_amdgcn_raw_buffer_load_b64(r, b, 0, 0);
}

}  // namespace tp
