// Host-only entry points of the C ABI: version, status names, trellis LUT.
#include "tp_common.h"

extern "C" int tp_abi_version(void) { return TP_ABI_VERSION; }

extern "C" const char* tp_status_string(int status) {
  switch (status) {
    case TP_OK: return "ok";
    case TP_ERR_NULL_POINTER: return "null pointer";
    case TP_ERR_UNSUPPORTED_BITS: return "unsupported bits per weight";
    case TP_ERR_UNSUPPORTED_STATES: return "unsupported trellis state count (need 4, 8, 16 or 64)";
    case TP_ERR_BAD_DIMS: return "bad dimensions";
    case TP_ERR_MISALIGNED: return "misaligned pointer or stride";
    case TP_ERR_BAD_BLOCK: return "bad Hadamard block (power of 2 dividing d, at most 16384)";
    case TP_ERR_HIP: return "HIP launch or runtime error";
    case TP_ERR_WORKSPACE: return "workspace missing or too small";
    case TP_ERR_BAD_LAYOUT: return "device layout does not match the call";
    default: return "unknown status";
  }
}

// subset_lut (runtime.py:106-119): LUT[x] = subset of the window x, computed
// from the window-coordinate generators (same function as the reference's
// reindexed subset_table lookup).
extern "C" int tp_subset_lut(int n_states, uint8_t* lut_out, int lut_len) {
  tp::TrellisTaps t;
  int st = tp::trellis_taps(n_states, &t);
  if (st) return st;
  if (!lut_out) return TP_ERR_NULL_POINTER;
  const int size = 1 << (t.m + 1);
  if (lut_len < size) return TP_ERR_BAD_DIMS;
  for (int x = 0; x < size; ++x) {
    uint32_t b0 = __builtin_popcount((uint32_t)x & t.g0w) & 1u;
    uint32_t b1 = __builtin_popcount((uint32_t)x & t.g1w) & 1u;
    lut_out[x] = (uint8_t)((b1 << 1) | b0);
  }
  return TP_OK;
}

// Streaming read of `n16` 16-byte words.  Every wave streams its own
// contiguous slice (a multiple of 64 words), eight 1 KiB loads in flight
// (short slices too: the loads past the slice are masked off):
// on MI355X this reads ~12 % faster than a grid-stride sweep of the same
// bytes (whose loads all land in one sliding window of the address space).
// XOR-folded so that nothing is elided; one word is stored only when the
// fold hits an arbitrary constant (practically never).
typedef uint32_t probe_v4 __attribute__((ext_vector_type(4)));
__global__ void __launch_bounds__(512) tp_read_probe_kernel(const probe_v4* __restrict__ p, uint64_t n16,
                                                            uint32_t* __restrict__ sink) {
  constexpr int U = 8;
  const int lane = threadIdx.x & 63;
  const uint64_t waves = (uint64_t)gridDim.x * (blockDim.x >> 6);
  const uint64_t w = (uint64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const uint64_t per = ((n16 + waves - 1) / waves + 63) & ~(uint64_t)63;
  const uint64_t lo = w * per;
  const uint64_t hi = lo + per < n16 ? lo + per : n16;
  probe_v4 acc = {0u, 0u, 0u, 0u};
  for (uint64_t i = lo; i < hi; i += 64 * U) {
    probe_v4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint64_t k = i + 64 * u + lane;
      v[u] = k < hi ? __builtin_nontemporal_load(p + k) : probe_v4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u];
  }
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9E3779B9u) sink[0] = 1u;
}

extern "C" int tp_read_probe(const void* buf, int64_t bytes, uint32_t* sink, void* stream) {
  if (!buf || !sink) return TP_ERR_NULL_POINTER;
  if (bytes < 16 || (bytes & 15)) return TP_ERR_BAD_DIMS;
  if ((uintptr_t)buf & 15) return TP_ERR_MISALIGNED;
  const int grid = 2 * tp::device_cu_count();  // 2 workgroups of 512 threads per CU
  hipLaunchKernelGGL(tp_read_probe_kernel, dim3(grid), dim3(512), 0, (hipStream_t)stream,
                     reinterpret_cast<const probe_v4*>(buf), (uint64_t)bytes / 16u, sink);
  return tp::launch_status();
}
