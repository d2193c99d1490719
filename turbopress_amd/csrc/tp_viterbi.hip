// TCQ Viterbi encoder (compress time): the minimum-distortion trellis path
// of each row, bit-exact with the reference's fp32 algorithm
// (turbopress/trellis.py:111-179, pipeline.py:209-276).
//
// One wave per row, lane s = trellis state s (S <= 64 states; lanes >= S
// idle).  Per column t:
//   * the row's value z_t is wave-uniform (scalar loads, 16 columns at once);
//   * each lane needs the cost of two subsets -- the labels of its two
//     incoming branches, fixed per state -- so it keeps those two subsets'
//     midpoint thresholds and member values in registers, counts the
//     thresholds below z_t (= torch.bucketize, right=False) and forms
//     (z_t - member)^2 in fp32;
//   * the predecessors' metrics come from two lane shuffles (states s>>1 and
//     (s>>1) | S/2), cand = metric + cost in fp32, the branch-1 candidate wins
//     only if strictly smaller (the reference's `cand1 < cand0`);
//   * the 64 branch decisions are one ballot, stored as a 64-bit word per
//     column in the caller's workspace.
// Floating-point contraction is off in this file: every add and multiply
// rounds separately, as torch's CPU ops do, so the metrics agree bit for bit.
// The end state is the first state of minimum metric (torch.argmin).  The
// backtrack walks the decisions from the end with scalar operations,
// collecting the state sequence 64 columns at a time into one register (a
// lane per column); the lanes then emit path bit, subset, member and level of
// their columns in parallel.
#pragma clang fp contract(off)

#include "tp_common.h"

namespace tp {
namespace {

constexpr int kVitWaves = 4;  // rows per workgroup

template <int NS>
struct Gen;
template <> struct Gen<4> { static constexpr int m = 2; static constexpr uint32_t g0 = 05, g1 = 07; };
template <> struct Gen<8> { static constexpr int m = 3; static constexpr uint32_t g0 = 015, g1 = 017; };
template <> struct Gen<16> { static constexpr int m = 4; static constexpr uint32_t g0 = 023, g1 = 035; };
template <> struct Gen<64> { static constexpr int m = 6; static constexpr uint32_t g0 = 0133, g1 = 0171; };

// Subset label of the branch from state `prev` on input bit b
// (trellis.py:73-80): x = (b << m) | prev, label = par(x & g1) << 1 | par(x & g0).
template <int NS>
__device__ __forceinline__ int branch_subset(int prev, int b) {
  const uint32_t x = ((uint32_t)b << Gen<NS>::m) | (uint32_t)prev;
  return (int)(((__popc(x & Gen<NS>::g1) & 1) << 1) | (__popc(x & Gen<NS>::g0) & 1));
}

// Member count of one subset at `bits` bits/weight: 2^(bits+1) levels / 4.
template <int BITS>
struct Sub {
  static constexpr int M = 1 << (BITS - 1);
  float thr[M > 1 ? M - 1 : 1];  // midpoints between consecutive members
  float val[M];                  // members, ascending (codebook[j::4])
};

template <int BITS>
__device__ __forceinline__ Sub<BITS> load_subset(const float* __restrict__ cb, int j) {
  Sub<BITS> s;
#pragma unroll
  for (int i = 0; i < Sub<BITS>::M; ++i) s.val[i] = cb[4 * i + j];
#pragma unroll
  for (int i = 0; i + 1 < Sub<BITS>::M; ++i) s.thr[i] = (s.val[i] + s.val[i + 1]) / 2.0f;
  return s;
}

// Nearest member (index = number of thresholds strictly below z) and its
// squared error.
// The member is selected by the comparisons themselves (thresholds ascend,
// so the last one below z names it).  Each candidate value passes through an
// empty asm statement first: a select between two loads of the struct would
// otherwise become a load through a selected address, i.e. a private-memory
// table lookup.
template <int BITS>
__device__ __forceinline__ float subset_cost(const Sub<BITS>& s, float z, int* member) {
  int m = 0;
  float v = s.val[0];
  __asm__("" : "+v"(v));
#pragma unroll
  for (int i = 0; i + 1 < Sub<BITS>::M; ++i) {
    const bool above = s.thr[i] < z;
    float next = s.val[i + 1];
    __asm__("" : "+v"(next));
    m += above ? 1 : 0;
    v = above ? next : v;
  }
  if (member) *member = m;
  const float diff = z - v;
  return diff * diff;
}

template <int NS, int BITS>
__global__ void __launch_bounds__(64 * kVitWaves)
viterbi_kernel(const float* __restrict__ z, int64_t ldz, int64_t n, int d, const float* __restrict__ cb,
               const int32_t* __restrict__ start_state, uint8_t* __restrict__ level, uint8_t* __restrict__ path,
               uint8_t* __restrict__ member, int32_t* __restrict__ end_state, uint64_t* __restrict__ bp_ws) {
  __shared__ float s_cb[4 * Sub<BITS>::M];
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kVitWaves + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  for (int i = threadIdx.x; i < 4 * Sub<BITS>::M; i += blockDim.x) s_cb[i] = cb[i];
  __syncthreads();
  if (row >= n) return;  // whole wave leaves together

  const float* zr = z + row * ldz;
  // wave-uniform reads of the row through the constant address space: scalar loads
  const __attribute__((address_space(4))) float* zc_row = (const __attribute__((address_space(4))) float*)zr;
  uint64_t* bp = bp_ws + row * (int64_t)d;
  const int s = lane < NS ? lane : 0;
  const int p0 = s >> 1, p1 = (s >> 1) | (NS >> 1);
  const int sub0 = branch_subset<NS>(p0, s & 1), sub1 = branch_subset<NS>(p1, s & 1);
  const Sub<BITS> S0 = load_subset<BITS>(s_cb, sub0);
  const Sub<BITS> S1 = load_subset<BITS>(s_cb, sub1);
  const int start = start_state ? start_state[row] : 0;
  float alpha = (lane == start) ? 0.0f : __builtin_inff();

  // ---- forward pass ----------------------------------------------------
  for (int t0 = 0; t0 < d; t0 += 16) {
    // (a full chunk is read whenever it fits; the tail reads column by column)
    float zc[16];
    if (t0 + 16 <= d) {
#pragma unroll
      for (int i = 0; i < 16; ++i) zc[i] = zc_row[t0 + i];
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) zc[i] = t0 + i < d ? zc_row[t0 + i] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (t0 + i >= d) continue;  // uniform; the loop still unrolls
      const float c0 = subset_cost<BITS>(S0, zc[i], nullptr);
      const float c1 = subset_cost<BITS>(S1, zc[i], nullptr);
      const float a0 = __shfl(alpha, p0, 64);
      const float a1 = __shfl(alpha, p1, 64);
      const float cand0 = a0 + c0;
      const float cand1 = a1 + c1;
      const bool take1 = lane < NS && cand1 < cand0;
      alpha = take1 ? cand1 : cand0;
      const uint64_t mask = __ballot(take1);
      if (lane == 0) bp[t0 + i] = mask;
    }
  }

  // ---- end state: first state of minimum metric -------------------------
  float mn = lane < NS ? alpha : __builtin_inff();
#pragma unroll
  for (int w = 1; w < 64; w <<= 1) mn = fminf(mn, __shfl_xor(mn, w, 64));
  const uint64_t at_min = __ballot(lane < NS && alpha == mn);
  // all metrics infinite (cannot happen from a finite start): state 0
  int state = at_min ? (int)__builtin_ctzll(at_min) : 0;
  if (lane == 0 && end_state) end_state[row] = state;

  // ---- backtrack, 64 columns per round ------------------------------------
  // bp must be visible to this wave's own scalar/vector reads below.
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  uint8_t* lr = level + row * (int64_t)d;
  uint8_t* pr = path + row * (int64_t)d;
  uint8_t* mr = member + row * (int64_t)d;
  const int last_base = ((d - 1) / 64) * 64;
  for (int tb = last_base; tb >= 0; tb -= 64) {
    // states after columns tb .. tb+63 (lane i <-> column tb + i), walked
    // from the highest column down; `state` is the state after column t.
    const int hi = min(63, d - 1 - tb);
    // the round's 64 decision words, one per lane, fetched together
    const uint64_t my_bp = lane <= hi ? bp[tb + lane] : 0;
    const uint32_t bp_lo = (uint32_t)my_bp, bp_hi = (uint32_t)(my_bp >> 32);
    int st_lane = 0;
    for (int i = hi; i >= 0; --i) {
      st_lane = lane == i ? state : st_lane;
      const uint64_t m = (uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)bp_lo, i) |
                         ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)bp_hi, i) << 32);
      const int take1 = (int)((m >> state) & 1u);
      state = take1 ? ((state >> 1) | (NS >> 1)) : (state >> 1);
    }
    if (lane <= hi) {
      const int t = tb + lane;
      const int take1 = (int)((my_bp >> st_lane) & 1u);
      const int prev = take1 ? ((st_lane >> 1) | (NS >> 1)) : (st_lane >> 1);
      const int sub = branch_subset<NS>(prev, st_lane & 1);
      const Sub<BITS> Ss = load_subset<BITS>(s_cb, sub);
      int mem = 0;
      (void)subset_cost<BITS>(Ss, zr[t], &mem);
      pr[t] = (uint8_t)(st_lane & 1);
      mr[t] = (uint8_t)mem;
      lr[t] = (uint8_t)(mem * 4 + sub);
    }
  }
}

template <int NS>
int launch_viterbi(int bits, const float* z, int64_t ldz, int64_t n, int d, const float* cb, const int32_t* start,
                   uint8_t* level, uint8_t* path, uint8_t* member, int32_t* end_state, uint64_t* ws,
                   hipStream_t s) {
  const dim3 grid((unsigned)((n + kVitWaves - 1) / kVitWaves)), block(64 * kVitWaves);
  switch (bits) {
    case 1: hipLaunchKernelGGL((viterbi_kernel<NS, 1>), grid, block, 0, s, z, ldz, n, d, cb, start, level, path, member, end_state, ws); break;
    case 2: hipLaunchKernelGGL((viterbi_kernel<NS, 2>), grid, block, 0, s, z, ldz, n, d, cb, start, level, path, member, end_state, ws); break;
    case 3: hipLaunchKernelGGL((viterbi_kernel<NS, 3>), grid, block, 0, s, z, ldz, n, d, cb, start, level, path, member, end_state, ws); break;
    case 4: hipLaunchKernelGGL((viterbi_kernel<NS, 4>), grid, block, 0, s, z, ldz, n, d, cb, start, level, path, member, end_state, ws); break;
    default: return TP_ERR_UNSUPPORTED_BITS;
  }
  return launch_status();
}

}  // namespace
}  // namespace tp

using namespace tp;

extern "C" int64_t tp_viterbi_workspace_bytes(int64_t n, int64_t d) {
  if (n <= 0 || d <= 0 || n > INT64_MAX / (int64_t)sizeof(uint64_t) / d) return 0;
  return n * d * (int64_t)sizeof(uint64_t);
}

extern "C" int tp_tcq_viterbi(const float* z, int64_t ldz, int64_t n, int64_t d, const float* codebook, int bits,
                              int n_states, const int32_t* start_state, uint8_t* level_codes, uint8_t* path_bits,
                              uint8_t* member_codes, int32_t* end_state, void* workspace, int64_t workspace_bytes,
                              void* stream) {
  if (!z || !codebook || !level_codes || !path_bits || !member_codes || !workspace) return TP_ERR_NULL_POINTER;
  if (bits < 1 || bits > 4) return TP_ERR_UNSUPPORTED_BITS;
  if (n <= 0 || d <= 0 || d > (1 << 24) || ldz < d || n > ((int64_t)1 << 36)) return TP_ERR_BAD_DIMS;
  if (workspace_bytes < tp_viterbi_workspace_bytes(n, d)) return TP_ERR_WORKSPACE;
  if (((uintptr_t)workspace & 7) || ((uintptr_t)z & 3) || ((uintptr_t)codebook & 3)) return TP_ERR_MISALIGNED;
  hipStream_t s = (hipStream_t)stream;
  uint64_t* ws = reinterpret_cast<uint64_t*>(workspace);
  switch (n_states) {
    case 4: return launch_viterbi<4>(bits, z, ldz, n, (int)d, codebook, start_state, level_codes, path_bits, member_codes, end_state, ws, s);
    case 8: return launch_viterbi<8>(bits, z, ldz, n, (int)d, codebook, start_state, level_codes, path_bits, member_codes, end_state, ws, s);
    case 16: return launch_viterbi<16>(bits, z, ldz, n, (int)d, codebook, start_state, level_codes, path_bits, member_codes, end_state, ws, s);
    case 64: return launch_viterbi<64>(bits, z, ldz, n, (int)d, codebook, start_state, level_codes, path_bits, member_codes, end_state, ws, s);
    default: return TP_ERR_UNSUPPORTED_STATES;
  }
}
