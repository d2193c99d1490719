// PackedTCQLinear forward for callers that cannot allocate device memory.
//
// tp_packed_linear_forward takes a caller-allocated split-K workspace (fp32
// partial sums and per-tile counters, used at batch 5..32).  Code under HIP
// graph capture, tight serving loops and harnesses that forbid hipMalloc
// cannot provide one; this variant uses a workspace of fixed maximum size
// that the library holds in a file-scope device array instead.  Each GPU
// holds its own copy of the array until the process ends; its address on a
// device is looked up once per device (hipGetSymbolAddress, with the device
// current) on the first call there, and only that address is ever handed to
// kernels or copies.  Every call on one GPU shares the array: calls that
// overlap on one GPU race.  Each launch that uses the array is preceded by
// a fill kernel that clears the bytes it uses, so a call does not depend on
// what the previous one left; launches that use none (the one-pass kernel
// without a K split) clear nothing.
#include "tp_tiled_common.h"

#include <algorithm>
#include <mutex>

namespace tp {

// Split-K sums + counters of tp_gemv_workspace_bytes(n, batch) for n up to
// 16384 rows at any batch <= 32 and 32768 rows at batch <= 16: T row tiles
// of 16 rows x 16 (batch <= 16) or 32 fp32 columns, plus T counters.
constexpr int64_t kNoAllocScratchBytes = 2 * 1024 * 1024 + 8192;
static_assert(kNoAllocScratchBytes % 16 == 0, "cleared in 16-byte words");
static_assert(kNoAllocScratchBytes >= (16384 / 16) * 16 * 32 * 4 + (16384 / 16) * 4, "16384 rows, batch 32");
static_assert(kNoAllocScratchBytes >= (32768 / 16) * 16 * 16 * 4 + (32768 / 16) * 4, "32768 rows, batch 16");

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mutex;
void* g_scratch_ptr[64];

// Device address of `scratch` on the current device (looked up once per device).
int scratch_address(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return TP_ERR_HIP;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return TP_ERR_HIP;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return TP_OK;
}

// Zero n4 4-byte words (a fill kernel rather than a memset node, so that a
// captured graph replays it like any other kernel).
__global__ void __launch_bounds__(256) zero_words_kernel(uint32_t* __restrict__ p, int64_t n4) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) p[i] = 0u;
}

int zero_device_bytes(void* p, int64_t bytes, hipStream_t s) {
  if (bytes <= 0) return TP_OK;
  if (!p || (bytes & 3) || ((uintptr_t)p & 3)) return TP_ERR_MISALIGNED;
  const int64_t n4 = bytes / 4;
  const int grid = (int)std::min<int64_t>((n4 + 255) / 256, 1024);
  hipLaunchKernelGGL(zero_words_kernel, dim3(grid), dim3(256), 0, s, reinterpret_cast<uint32_t*>(p), n4);
  return launch_status();
}

}  // namespace tp

using namespace tp;

extern "C" int tp_packed_linear_forward_noalloc(const uint16_t* x, int64_t ldx, int64_t batch,
                                                const uint16_t* rot_scale, int64_t block,
                                                const uint8_t* path_tiled, const uint8_t* member_tiled,
                                                const uint16_t* scales, const uint16_t* codebook,
                                                const uint16_t* bias, int64_t n, int64_t d, int bits,
                                                int n_states, uint16_t* y, int64_t ldy, void* stream) {
  if (batch < 1 || batch > 32 || n <= 0 || d <= 0) return TP_ERR_BAD_DIMS;
  void* ws = nullptr;
  const int st = scratch_address(&ws);
  if (st) return st;
  // The route is chosen as for tp_packed_linear_forward with the whole array
  // as workspace; a route whose workspace would exceed it returns
  // TP_ERR_WORKSPACE before any launch, and each launch that uses it is
  // preceded by a fill of the bytes it uses.
  return packed_linear_forward_cleared(x, ldx, batch, rot_scale, block, path_tiled, member_tiled, scales, codebook,
                                       bias, n, d, bits, n_states, y, ldy, ws, kNoAllocScratchBytes, stream);
}
