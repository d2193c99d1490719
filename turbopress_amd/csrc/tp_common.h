// Shared definitions for the turbopress_amd HIP kernels (gfx950 / CDNA4).
//
// Trellis conventions (reference: turbopress/trellis.py:47-80,
// turbopress/runtime.py:106-139):
//   * the path stream holds one bit b[t] per weight; the "window" of weight t
//     is the (m+1)-bit little-endian field x = sum_j b[t-m+j] << j, with
//     b[<0] = 0 at each row start (m = log2 S);
//   * subset(t) = (parity(x & G1w) << 1) | parity(x & G0w), where G0w/G1w
//     are the convolutional generators re-expressed in window coordinates
//     (the low m generator bits reversed, bit m kept) -- this is exactly the
//     reference's subset_lut(trellis)[x] without a table;
//   * level(t) = member(t) * 4 + subset(t); weight = codebook[level].
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <mutex>
#include <set>
#include <utility>

#include "../../include/turbopress_amd.h"

namespace tp {

// Octal generators per state count (trellis.py:47-52).
inline int generators(int n_states, uint32_t* g0, uint32_t* g1) {
  switch (n_states) {
    case 4: *g0 = 05; *g1 = 07; return 2;
    case 8: *g0 = 015; *g1 = 017; return 3;
    case 16: *g0 = 023; *g1 = 035; return 4;
    case 64: *g0 = 0133; *g1 = 0171; return 6;
    default: return -1;
  }
}

// Generator g (over x' = (b << m) | state) rewritten over the stream window.
inline uint32_t window_generator(uint32_t g, int m) {
  uint32_t w = ((g >> m) & 1u) << m;
  for (int j = 0; j < m; ++j) w |= ((g >> (m - 1 - j)) & 1u) << j;
  return w;
}

struct TrellisTaps {
  int m;          // log2(n_states)
  uint32_t g0w;   // window-coordinate generator for subset bit 0
  uint32_t g1w;   // window-coordinate generator for subset bit 1
};

inline int trellis_taps(int n_states, TrellisTaps* t) {
  uint32_t g0, g1;
  int m = generators(n_states, &g0, &g1);
  if (m < 0) return TP_ERR_UNSUPPORTED_STATES;
  t->m = m;
  t->g0w = window_generator(g0, m);
  t->g1w = window_generator(g1, m);
  return TP_OK;
}

__device__ __forceinline__ uint32_t subset_of_window(uint32_t x, uint32_t g0w, uint32_t g1w) {
  return ((__popc(x & g1w) & 1u) << 1) | (__popc(x & g0w) & 1u);
}

// Little-endian bit-field read of `width` (<= 25) bits starting at stream bit
// `bit` of a byte row; bytes at or beyond `row_bytes` read as zero.
__device__ __forceinline__ uint32_t read_bits_le(const uint8_t* row, int64_t row_bytes,
                                                 int64_t bit, int width) {
  int64_t byte0 = bit >> 3;
  uint32_t v = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int64_t b = byte0 + i;
    uint32_t byte = (b < row_bytes) ? (uint32_t)row[b] : 0u;
    v |= byte << (8 * i);
  }
  return (v >> (bit & 7)) & ((1u << width) - 1u);
}

// Path window of weight t in a row: bits b[t-m .. t], zero before the row.
__device__ __forceinline__ uint32_t path_window(const uint8_t* row, int64_t row_bytes,
                                                int64_t t, int m) {
  int64_t lo = t - m;
  if (lo >= 0) return read_bits_le(row, row_bytes, lo, m + 1);
  // Row start: only bits 0..t exist; they land at window bits (m-t)..m.
  uint32_t v = read_bits_le(row, row_bytes, 0, (int)(t + 1));
  return v << (uint32_t)(-lo);
}

__device__ __forceinline__ float h2f(uint16_t h) {
  return __half2float(__ushort_as_half(h));
}

__device__ __forceinline__ uint16_t f2h(float f) {
  return __half_as_ushort(__float2half_rn(f));
}

inline int check_bits(int bits) {
  return (bits >= 1 && bits <= 7) ? TP_OK : TP_ERR_UNSUPPORTED_BITS;
}

// CUs of the current device (cached per device; 256 if the query fails).
inline int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

// Largest LDS allocation of one workgroup on the current device (cached per
// device; 64 KiB if the query fails).
inline int device_max_lds() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 64 * 1024;
  if (!cached[dev]) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0)
      v = 64 * 1024;
    cached[dev] = v;
  }
  return cached[dev];
}

// Let kernel `fn` (with `static_bytes` of static LDS) take the rest of the
// device's LDS as dynamic LDS.  Done once per kernel and device; later
// launches make no runtime call for it.
inline void allow_dynamic_lds(const void* fn, int static_bytes) {
  static std::mutex mu;
  static std::set<std::pair<const void*, int>> done;
  int dev = 0;
  (void)hipGetDevice(&dev);
  std::lock_guard<std::mutex> lock(mu);
  if (done.insert({fn, dev}).second)
    (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, device_max_lds() - static_bytes);
}

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? TP_OK : TP_ERR_HIP;
}

}  // namespace tp
