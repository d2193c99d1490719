// Window decode and generic GEMV over the natural format-v2 streams.
//
// Reference semantics:
//   * window_decode_levels  turbopress/runtime.py:122-139 (+ unpack_le :93-100)
//   * decode_rows           turbopress/runtime.py:291-301
//   * packed GEMV           turbopress/triton_kernel.py:44-157 (row scale
//                           factored out of an fp32 reduction, fp16 output)
//                           then the fp16 bias add of runtime.py:332-333.
//
// These kernels read the streams exactly as the reference stores them (one
// weight per thread, byte-granular little-endian field reads), support every
// bits in [1, 7] and every S in {4, 8, 16, 64}, and serve as the bit-exact
// decode entry points and the general fallback GEMV.  The bandwidth-tuned
// path for k in {2, 3, 4} lives in tp_gemv_tiled.hip.
#include "tp_common.h"

namespace tp {

struct DecodeArgs {
  const uint8_t* path;
  int64_t path_stride;
  const uint8_t* member;
  int64_t member_stride;
  int64_t n_rows;
  int64_t d;
  int bits;
  int m;
  uint32_t g0w, g1w;
};

__device__ __forceinline__ uint32_t level_at(const DecodeArgs& a, int64_t r, int64_t c) {
  const uint8_t* prow = a.path + r * a.path_stride;
  uint32_t win = path_window(prow, a.path_stride, c, a.m);
  uint32_t sub = subset_of_window(win, a.g0w, a.g1w);
  uint32_t mem = 0;
  if (a.bits > 1) {
    const uint8_t* mrow = a.member + r * a.member_stride;
    mem = read_bits_le(mrow, a.member_stride, c * (a.bits - 1), a.bits - 1);
  }
  return mem * 4u + sub;
}

__global__ void window_decode_kernel(DecodeArgs a, uint8_t* __restrict__ out, int64_t out_stride) {
  const int64_t r = blockIdx.y;
  for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < a.d;
       c += (int64_t)gridDim.x * blockDim.x) {
    out[r * out_stride + c] = (uint8_t)level_at(a, r, c);
  }
}

__global__ void decode_rows_kernel(DecodeArgs a, const uint16_t* __restrict__ scales,
                                   const uint16_t* __restrict__ codebook,
                                   uint16_t* __restrict__ out, int64_t out_stride) {
  const int64_t r = blockIdx.y;
  const float sc = h2f(scales[r]);
  for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < a.d;
       c += (int64_t)gridDim.x * blockDim.x) {
    // fp32 product of two fp16 values is exact; one rounding to fp16.
    out[r * out_stride + c] = f2h(h2f(codebook[level_at(a, r, c)]) * sc);
  }
}

// One wave per output row; lanes stride over the columns; the batch is
// processed in chunks of 8 accumulators.
constexpr int kGenericBatchChunk = 8;

__global__ void __launch_bounds__(256)
generic_gemv_kernel(DecodeArgs a, const uint16_t* __restrict__ z, int64_t batch,
                    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ codebook,
                    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int64_t n) {
  __shared__ float cb[256];
  const int ncb = 1 << (a.bits + 1);
  for (int i = threadIdx.x; i < ncb; i += blockDim.x) cb[i] = h2f(codebook[i]);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
  if (r >= n) return;
  const float sc = h2f(scales[r]);
  for (int64_t b0 = 0; b0 < batch; b0 += kGenericBatchChunk) {
    const int nb = (int)((batch - b0) < kGenericBatchChunk ? (batch - b0) : kGenericBatchChunk);
    float acc[kGenericBatchChunk];
#pragma unroll
    for (int b = 0; b < kGenericBatchChunk; ++b) acc[b] = 0.f;
    for (int64_t c = lane; c < a.d; c += 64) {
      const float w = cb[level_at(a, r, c)];
#pragma unroll
      for (int b = 0; b < kGenericBatchChunk; ++b)
        if (b < nb) acc[b] += w * h2f(z[(b0 + b) * a.d + c]);
    }
#pragma unroll
    for (int b = 0; b < kGenericBatchChunk; ++b) {
      float v = acc[b];
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
      acc[b] = v;
    }
    if (lane == 0) {
      for (int b = 0; b < nb; ++b) {
        uint16_t out = f2h(acc[b] * sc);
        if (bias) out = f2h(h2f(out) + h2f(bias[r]));
        y[(b0 + b) * n + r] = out;
      }
    }
  }
}

inline int make_decode_args(const uint8_t* path, int64_t path_stride, const uint8_t* member,
                            int64_t member_stride, int64_t n_rows, int64_t d, int bits,
                            int n_states, DecodeArgs* a) {
  if (!path) return TP_ERR_NULL_POINTER;
  int st = check_bits(bits);
  if (st) return st;
  if (bits > 1 && !member) return TP_ERR_NULL_POINTER;
  TrellisTaps taps;
  st = trellis_taps(n_states, &taps);
  if (st) return st;
  if (n_rows < 0 || d <= 0) return TP_ERR_BAD_DIMS;
  if (path_stride < (d + 7) / 8) return TP_ERR_BAD_DIMS;
  if (bits > 1 && member_stride < (d * (bits - 1) + 7) / 8) return TP_ERR_BAD_DIMS;
  a->path = path;
  a->path_stride = path_stride;
  a->member = member;
  a->member_stride = member_stride;
  a->n_rows = n_rows;
  a->d = d;
  a->bits = bits;
  a->m = taps.m;
  a->g0w = taps.g0w;
  a->g1w = taps.g1w;
  return TP_OK;
}

inline dim3 decode_grid(int64_t n_rows, int64_t d) {
  int64_t bx = (d + 255) / 256;
  if (bx > 64) bx = 64;
  return dim3((unsigned)bx, (unsigned)n_rows);
}

}  // namespace tp

extern "C" int tp_window_decode_levels(const uint8_t* path, int64_t path_stride,
                                       const uint8_t* member, int64_t member_stride,
                                       int64_t n_rows, int64_t d, int bits, int n_states,
                                       uint8_t* levels_out, int64_t out_stride, void* stream) {
  using namespace tp;
  DecodeArgs a;
  int st = make_decode_args(path, path_stride, member, member_stride, n_rows, d, bits, n_states, &a);
  if (st) return st;
  if (!levels_out) return TP_ERR_NULL_POINTER;
  if (out_stride < d) return TP_ERR_BAD_DIMS;
  if (n_rows == 0) return TP_OK;
  if (n_rows > 65535) return TP_ERR_BAD_DIMS;
  hipLaunchKernelGGL(window_decode_kernel, decode_grid(n_rows, d), dim3(256), 0,
                     (hipStream_t)stream, a, levels_out, out_stride);
  return launch_status();
}

extern "C" int tp_decode_rows(const uint8_t* path, int64_t path_stride,
                              const uint8_t* member, int64_t member_stride,
                              const uint16_t* scales, const uint16_t* codebook,
                              int64_t n_rows, int64_t d, int bits, int n_states,
                              uint16_t* w_out, int64_t out_stride, void* stream) {
  using namespace tp;
  DecodeArgs a;
  int st = make_decode_args(path, path_stride, member, member_stride, n_rows, d, bits, n_states, &a);
  if (st) return st;
  if (!scales || !codebook || !w_out) return TP_ERR_NULL_POINTER;
  if (out_stride < d) return TP_ERR_BAD_DIMS;
  if (n_rows == 0) return TP_OK;
  if (n_rows > 65535) return TP_ERR_BAD_DIMS;
  hipLaunchKernelGGL(decode_rows_kernel, decode_grid(n_rows, d), dim3(256), 0,
                     (hipStream_t)stream, a, scales, codebook, w_out, out_stride);
  return launch_status();
}

extern "C" int tp_tcq_gemv(const uint16_t* z, int64_t batch,
                           const uint8_t* path, int64_t path_stride,
                           const uint8_t* member, int64_t member_stride,
                           const uint16_t* scales, const uint16_t* codebook, const uint16_t* bias,
                           int64_t n, int64_t d, int bits, int n_states,
                           uint16_t* y, void* stream) {
  using namespace tp;
  DecodeArgs a;
  int st = make_decode_args(path, path_stride, member, member_stride, n, d, bits, n_states, &a);
  if (st) return st;
  if (!z || !scales || !codebook || !y) return TP_ERR_NULL_POINTER;
  if (batch < 0) return TP_ERR_BAD_DIMS;
  if (batch == 0 || n == 0) return TP_OK;
  const int rows_per_block = 4;
  dim3 grid((unsigned)((n + rows_per_block - 1) / rows_per_block));
  hipLaunchKernelGGL(generic_gemv_kernel, grid, dim3(64 * rows_per_block), 0,
                     (hipStream_t)stream, a, z, batch, scales, codebook, bias, y, n);
  return launch_status();
}
