// Randomized-Hadamard activation rotation: z = blockFWHT(x * rot_scale).
//
// Reference semantics: turbopress/runtime.py:192-208 (_fwht/_block_fwht, the
// orthonormal Sylvester transform in natural order, butterflies at distance
// h = 1, 2, 4, ... then one division by sqrt(block)) applied to
// x.f32 * rot_scale.f32 (runtime.py:323), i.e. the fp32 CPU path; the fused
// reference kernel (triton_kernel.py:172-212) computes the same transform with
// fp16 intermediates.  Here every stage is fp32 and z is rounded to fp16 once.
//
// One workgroup transforms one block of one batch row.  The block lives in
// LDS as fp32 (block <= 16384 -> 64 KiB).  The first log2(EPT) stages run in
// registers (each thread owns EPT consecutive elements), the rest exchange
// through LDS with one barrier per stage.
#include "tp_common.h"

namespace tp {

constexpr int kRotMaxBlock = 16384;

template <int EPT>
__global__ void __launch_bounds__(256)
fwht_scale_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ rs,
                  const uint16_t* __restrict__ post, uint16_t* __restrict__ z, int64_t d,
                  int64_t ldz, int block, float inv_norm_div) {
  extern __shared__ float buf[];
  const int64_t row = blockIdx.y;
  const int64_t base = (int64_t)blockIdx.x * block;
  const uint16_t* xr = x + row * d + base;
  const uint16_t* rr = rs ? rs + base : nullptr;
  const uint16_t* pr = post ? post + base : nullptr;
  uint16_t* zr = z + row * ldz + base;
  const int nchunks = block / EPT;  // EPT-element chunks, one per thread per pass
  const int t = threadIdx.x;

  for (int c = t; c < nchunks; c += blockDim.x) {
    float v[EPT];
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      v[e] = h2f(xr[c * EPT + e]);
      if (rr) v[e] *= h2f(rr[c * EPT + e]);
    }
    // In-register stages h = 1 .. EPT/2 (natural order, a+b then a-b).
#pragma unroll
    for (int h = 1; h < EPT; h <<= 1) {
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        if ((e & h) == 0) {
          float a = v[e], b = v[e + h];
          v[e] = a + b;
          v[e + h] = a - b;
        }
      }
    }
#pragma unroll
    for (int e = 0; e < EPT; ++e) buf[c * EPT + e] = v[e];
  }
  __syncthreads();
  // Cross-thread stages h = EPT .. block/2 through LDS.
  for (int h = EPT; h < block; h <<= 1) {
    for (int i = t; i < block / 2; i += blockDim.x) {
      int j = (i / h) * (2 * h) + (i % h);
      float a = buf[j], b = buf[j + h];
      buf[j] = a + b;
      buf[j + h] = a - b;
    }
    __syncthreads();
  }
  for (int i = t; i < block; i += blockDim.x) {
    float v = buf[i] / inv_norm_div;
    if (pr) v *= h2f(pr[i]);
    zr[i] = f2h(v);
  }
  // The last block of a row also clears the padding columns [d, ldz).
  if (blockIdx.x == gridDim.x - 1) {
    uint16_t* zp = z + row * ldz;
    for (int64_t i = d + t; i < ldz; i += blockDim.x) zp[i] = 0;
  }
}

}  // namespace tp

namespace tp {

int block_fwht(const uint16_t* x, const uint16_t* pre, const uint16_t* post, uint16_t* z,
               int64_t rows, int64_t d, int64_t block, int64_t ldz, void* stream) {
  if (!x || !z) return TP_ERR_NULL_POINTER;
  if (rows < 0 || d <= 0 || ldz < d) return TP_ERR_BAD_DIMS;
  if (block < 1 || (block & (block - 1)) || d % block || block > kRotMaxBlock) return TP_ERR_BAD_BLOCK;
  if (rows == 0) return TP_OK;
  if (rows > 65535) return TP_ERR_BAD_DIMS;
  const int ept = block >= 8 ? 8 : (int)block;
  const int nchunks = (int)(block / ept);
  const int threads = nchunks < 256 ? (nchunks < 64 ? 64 : nchunks) : 256;
  dim3 grid((unsigned)(d / block), (unsigned)rows);
  // Division by the fp32 value of sqrt(block), as the reference divides an
  // fp32 tensor by math.sqrt(d).
  const float div = (float)__builtin_sqrt((double)block);
  const size_t lds = (size_t)block * sizeof(float);
  hipStream_t s = (hipStream_t)stream;
  switch (ept) {
    case 8: hipLaunchKernelGGL(fwht_scale_kernel<8>, grid, dim3(threads), lds, s, x, pre, post, z, d, ldz, (int)block, div); break;
    case 4: hipLaunchKernelGGL(fwht_scale_kernel<4>, grid, dim3(threads), lds, s, x, pre, post, z, d, ldz, (int)block, div); break;
    case 2: hipLaunchKernelGGL(fwht_scale_kernel<2>, grid, dim3(threads), lds, s, x, pre, post, z, d, ldz, (int)block, div); break;
    default: hipLaunchKernelGGL(fwht_scale_kernel<1>, grid, dim3(threads), lds, s, x, pre, post, z, d, ldz, (int)block, div); break;
  }
  return launch_status();
}

}  // namespace tp

extern "C" int tp_fwht_scale(const uint16_t* x, const uint16_t* rot_scale, uint16_t* z,
                             int64_t batch, int64_t d, int64_t block, void* stream) {
  if (!rot_scale) return TP_ERR_NULL_POINTER;
  return tp::block_fwht(x, rot_scale, nullptr, z, batch, d, block, d, stream);
}

extern "C" int tp_fwht_scale_padded(const uint16_t* x, const uint16_t* rot_scale, uint16_t* z,
                                    int64_t batch, int64_t d, int64_t block, int64_t ldz,
                                    void* stream) {
  if (!rot_scale) return TP_ERR_NULL_POINTER;
  return tp::block_fwht(x, rot_scale, nullptr, z, batch, d, block, ldz, stream);
}

extern "C" int tp_block_fwht_rows(const uint16_t* x, const uint16_t* pre_scale,
                                  const uint16_t* post_scale, uint16_t* out,
                                  int64_t rows, int64_t d, int64_t block, void* stream) {
  return tp::block_fwht(x, pre_scale, post_scale, out, rows, d, block, d, stream);
}
