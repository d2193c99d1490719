// Bandwidth path: device ("tiled") layout of the packed streams and the
// MFMA decode-GEMV that reads it.
//
// Device layout (exactly k bits per weight plus zero padding; a bijective
// re-arrangement of the reference's format-v2 streams, turbopress/runtime.py:73-100):
//   * rows are grouped in tiles of 16, columns in segments of 64; the number
//     of segments G is padded to a multiple of 4 (one "unit" = 4 segments);
//   * path words  [T][G][16 rows][2]:  X0, X1 with
//        X_x bit 2j   = path bit of column 64g + 16x + j        (first half)
//        X_x bit 2j+1 = path bit of column 64g + 32 + 16x + j   (second half)
//   * member words [T][G][16 rows][MW]:
//        k=3: M[x][h] (x = 0,1; h = first/second half), bits 2j..2j+1 = member
//             of column 64g + 32h + 16x + j (the reference's own bit order),
//             then the two nibbles of every byte swapped;
//        k=2: W[x], bits 4p..4p+1 = members of columns 64g + 16x + 2p, +1 and
//             bits 4p+2..4p+3 = members of columns 64g + 32 + 16x + 2p, +1;
//        k=4: the k=3 words of the low two member bits, then one word per
//             path word x of the high member bits, laid out for the
//             decoder's lane-offset bytes (see high_member_word) (MW = 6).
//
// Decode (per lane, 32 weights per path word; reference contract
// turbopress/runtime.py:122-139): the subset bits are parities of the path
// window with the trellis generators, i.e. XORs of the path stream delayed by
// each generator tap.  On the interleaved word a delay of t columns is a left
// funnel shift by 2t bits across (current word, previous word), so both
// subset bits of 32 weights cost ~12 ALU ops.  Two weights' (subset, member)
// bits form one byte (one bit-select per four bytes) that indexes a
// 256-entry table of fp16 pairs (cb[level_a], cb[level_b]); the table is
// replicated in LDS (k=3: two index formats x 32 lane copies, k=2: 64
// copies) so the lanes of a half-wave read distinct banks.  The pairs feed
// v_mfma_f32_16x16x32_f16 (rows x K) against the rotated activations (K x batch).
// The row scale is applied once at the end (turbopress/triton_kernel.py:70-73,123).
#include "tp_tiled_common.h"

#include <algorithm>

namespace tp {

struct GemvArgs {
  LinearDesc lin[kMaxInlineLinears];
  int32_t n_lin;
  int32_t total_blocks;
  int32_t batch;
  const uint16_t* codebook;
};

// ---------------------------------------------------------------------------
// GEMV kernel: persistent workgroups of 8 waves walk the block list; a block
// is (8 consecutive row tiles, kg <= 2 units along K); wave w takes tile w.
// Per block the workgroup stages the block's K range of z in LDS (rotating
// x on the fly when ROT), then every wave streams its tile.
// ---------------------------------------------------------------------------
template <int KB, int NS, int NBT, bool ROT>
__global__ void __launch_bounds__(kGroupThreads, 2)
tcq_gemv_tiled_kernel(const GemvArgs a) {
  // Static table (LDS address 0, so lookups fold the base into the
  // instruction offset) followed by the dynamic z staging area.
  __shared__ __attribute__((aligned(16))) uint32_t table[kTableWords];
  extern __shared__ __attribute__((aligned(16))) uint16_t zl[];
  constexpr int MW = member_words(KB);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r = lane & 15;   // A row / B,D column (batch)
  const int q = lane >> 4;   // K block of A and B, row block of D
  const uint32_t laneoff = lane_offsets<KB>(lane);
  const int batch = a.batch;
  bool table_ready = false;
  const uint32_t cb_lane = a.codebook[lane & ((2 << KB) - 1)];

  // One block.  The first call (the workgroup's first block) is a copy of
  // its own, so that its loads are scheduled from the kernel's entry state
  // rather than from the merged state of a loop: at the loop head the weight
  // loads waited for every earlier load, the codebook load included.
  auto block = [&](const int blk) __attribute__((always_inline)) {
    int li = 0, base = 0;
#pragma unroll
    for (int i = 0; i < kMaxInlineLinears - 1; ++i) {
      if (li + 1 < a.n_lin && blk >= base + a.lin[li].blocks) {
        base += a.lin[li].blocks;
        ++li;
      }
    }
    const LinearDesc& L = a.lin[li];
    const int rel = blk - base;
    const int nkb = (L.G4 + L.kg - 1) / L.kg;
    const int tb = rel / nkb, kb = rel - tb * nkb;
    const int t = tb * kWavesPerGroup + wave;
    const bool active = t < L.T;
    const int gu0 = kb * L.kg;
    const int ngu = min(L.kg, L.G4 - gu0);

    const uint32_t* pt = L.path + (size_t)(active ? t : 0) * L.G * (kTileRows * 2);
    const uint32_t* mt = L.member + (size_t)(active ? t : 0) * L.G * (kTileRows * MW);

    // Every load the block needs is issued here, before its LDS work: the
    // path/member words of all its units, the halo word, and (for the
    // common small case) the activations this wave stages.
    uint32_t x1_last = 0;
    uint2 X[kMaxUnitsPerBlock];
    uint32_t Mw[kMaxUnitsPerBlock][MW];
#pragma unroll
    for (int u = 0; u < kMaxUnitsPerBlock; ++u) {
      X[u] = uint2{0u, 0u};
#pragma unroll
      for (int i = 0; i < MW; ++i) Mw[u][i] = 0;
    }
    if (active) {
      if (gu0 > 0) x1_last = gld_w<MW>(pt + ((4 * gu0 - 1) * kTileRows + r) * 2 + 1);
#pragma unroll
      for (int u = 0; u < kMaxUnitsPerBlock; ++u) {
        if (u < ngu) {
          const int g = 4 * (gu0 + u) + q;
          X[u] = gld2_w<MW>(pt + (g * kTileRows + r) * 2);
#pragma unroll
          for (int i = 0; i < MW; ++i) Mw[u][i] = gld_w<MW>(mt + (g * kTileRows + r) * MW + i);
        }
      }
    }
    const ZPrefetch zp = prefetch_z<ROT>(L, gu0, ngu, batch, wave, lane);
    const bool small = ngu * batch <= kWavesPerGroup && (!ROT || L.hb <= 2 * kChunkCols);

    __syncthreads();  // every wave is done reading the previous block's z
    if (!table_ready) {
      build_pair_table_lanes<KB>(table, cb_lane, tid, kGroupThreads);
      table_ready = true;
    }
    if (small) {
      if (zp.valid) stage_z_prefetched<ROT>(L, gu0, batch, zl, wave, lane, zp);
    } else {
      stage_z<ROT>(L, gu0, ngu, batch, zl, wave, lane);
    }
    __syncthreads();
    if (!active) return;

    float4_t acc[NBT];
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt) acc[bt] = float4_t{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int u = 0; u < kMaxUnitsPerBlock; ++u) {
      if (u >= ngu) break;
      const int gu = gu0 + u;
      process_unit<KB, NS, NBT>(X[u], Mw[u], x1_last, gu, (4 * gu + q - 4 * gu0) * kSegCols, q, r,
                                lane, laneoff, table, zl, batch, acc);
      x1_last = X[u].y;
    }

    // Epilogue.  Lane holds D[4q + i][r]: rows 4q..4q+3 of the tile for batch column r.
    const int ldws = 16 * NBT;
    const int row0 = t * kTileRows + 4 * q;
    float sc[4], bs[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = min(row0 + i, L.n - 1);
      sc[i] = h2f(L.scales[row]);
      bs[i] = L.bias ? h2f(L.bias[row]) : 0.f;
    }
    if (ngu == L.G4) {
#pragma unroll
      for (int bt = 0; bt < NBT; ++bt) {
        const int nb = bt * 16 + r;
        if (nb >= batch) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (row0 + i >= L.n) continue;
          uint16_t out = f2h(acc[bt][i] * sc[i]);
          if (L.bias) out = f2h(h2f(out) + bs[i]);
          L.y[(size_t)nb * L.ldy + row0 + i] = out;
        }
      }
    } else {
      // Split K: partial sums travel only through device-scope read-modify-write
      // atomics, which are performed at the point of coherence, so waiting for
      // their completion orders them before the counter update without any
      // cache write-back or invalidation.
#pragma unroll
      for (int bt = 0; bt < NBT; ++bt) {
        const int nb = bt * 16 + r;
        if (nb >= batch) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          atomicAdd(L.ws + (size_t)(row0 + i) * ldws + bt * 16 + r, acc[bt][i]);
      }
      __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
      uint32_t old = 0;
      if (lane == 0) old = atomicAdd(L.cnt + t, (uint32_t)ngu);
      old = (uint32_t)__shfl((int)old, 0, 64);
      if (old + (uint32_t)ngu == (uint32_t)L.G4) {
        // Last contributor: read-and-clear the sums (also RMW atomics).
        float v[NBT][4];
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            v[bt][i] = (bt * 16 + r < batch)
                           ? atomicExch(L.ws + (size_t)(row0 + i) * ldws + bt * 16 + r, 0.f)
                           : 0.f;
        }
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) {
          const int nb = bt * 16 + r;
          if (nb >= batch) continue;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (row0 + i >= L.n) continue;
            uint16_t out = f2h(v[bt][i] * sc[i]);
            if (L.bias) out = f2h(h2f(out) + bs[i]);
            L.y[(size_t)nb * L.ldy + row0 + i] = out;
          }
        }
        if (lane == 0) atomicExch(L.cnt + t, 0u);
      }
    }
  };
  block((int)blockIdx.x);
  for (int blk = (int)(blockIdx.x + gridDim.x); blk < a.total_blocks; blk += (int)gridDim.x) block(blk);
}

// ---------------------------------------------------------------------------
// Debug decode of the tiled layout through the GEMV's own decode path:
// w[row, col] = fp16(f32(pair value) * f32(scale[row])).  One wave per unit.
// ---------------------------------------------------------------------------
template <int KB, int NS>
__global__ void __launch_bounds__(256)
tiled_decode_kernel(const uint32_t* __restrict__ path, const uint32_t* __restrict__ member,
                    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ cb,
                    int n, int d, int T, int G, int G4, uint16_t* __restrict__ w, int64_t ldw) {
  __shared__ uint32_t table[kTableWords];
  constexpr int MW = member_words(KB);
  build_pair_table<KB>(table, cb, threadIdx.x, blockDim.x);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int r = lane & 15, q = lane >> 4;
  const uint32_t laneoff = lane_offsets<KB>(lane);
  const int64_t unit = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (unit >= (int64_t)T * G4) return;
  const int t = (int)(unit / G4), gu = (int)(unit % G4);
  const int g = 4 * gu + q;
  const uint32_t* pt = path + (size_t)t * G * (kTileRows * 2);
  const uint32_t* mt = member + (size_t)t * G * (kTileRows * MW);
  const uint2 X = *reinterpret_cast<const uint2*>(pt + (g * kTileRows + r) * 2);
  const uint32_t halo = g > 0 ? pt[((g - 1) * kTileRows + r) * 2 + 1] : 0u;
  const uint32_t P = ((halo >> 1) & 0x55555555u) | ((X.y << 1) & 0xAAAAAAAAu);
  uint32_t Mw[MW];
  for (int i = 0; i < MW; ++i) Mw[i] = mt[(g * kTileRows + r) * MW + i];
  MemberWords<KB> mm[2];
  split_members<KB>(Mw, mm);
  const int row = t * kTileRows + r;
  const float sc = row < n ? h2f(scales[row]) : 0.f;
  for (int x = 0; x < 2; ++x) {
    u32x4_t A[4];
    decode_word<KB, NS>(x ? X.y : X.x, x ? X.x : P, mm[x], table, laneoff, A);
    if (row >= n) continue;
    for (int j = 0; j < 4; ++j) {
      for (int v = 0; v < 4; ++v) {
        for (int e = 0; e < 2; ++e) {
          const int col = g * kSegCols + (j >> 1) * 32 + 16 * x + 8 * (j & 1) + 2 * v + e;
          if (col >= d) continue;
          const uint16_t h = (uint16_t)(A[j][v] >> (16 * e));
          w[(int64_t)row * ldw + col] = f2h(h2f(h) * sc);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Re-tiling: natural format v2 streams -> device layout.  One thread per
// (tile, segment, row).  Columns past d and rows past n are zero.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t interleave16(uint32_t a, uint32_t b) {
  uint32_t o = 0;
  for (int j = 0; j < 16; ++j) o |= (((a >> j) & 1u) << (2 * j)) | (((b >> j) & 1u) << (2 * j + 1));
  return o;
}

__device__ __forceinline__ uint32_t pair_interleave16(uint32_t a, uint32_t b) {
  uint32_t o = 0;
  for (int p = 0; p < 8; ++p) o |= (((a >> (2 * p)) & 3u) << (4 * p)) | (((b >> (2 * p)) & 3u) << (4 * p + 2));
  return o;
}

// k=4 high member bits of path word x (first-half column group f, second
// half s; bit j = column j of the group), placed where the decoder moves
// them into bits 6..7 of each lane-offset byte: byte k holds columns 4k, 4k+1
// of f at bits 6, 7, columns 4k+2, 4k+3 of f at bits 4, 5, columns 4k, 4k+1
// of s at bits 2, 3 and columns 4k+2, 4k+3 of s at bits 0, 1.
__device__ __forceinline__ uint32_t high_member_word(uint32_t f, uint32_t s) {
  uint32_t o = 0;
  for (int k = 0; k < 4; ++k) {
    const uint32_t fb = (f >> (4 * k)) & 15u, sb = (s >> (4 * k)) & 15u;
    o |= ((fb & 3u) << (8 * k + 6)) | (((fb >> 2) & 3u) << (8 * k + 4)) | ((sb & 3u) << (8 * k + 2)) |
         (((sb >> 2) & 3u) << (8 * k));
  }
  return o;
}

__device__ __forceinline__ uint32_t nibble_swap(uint32_t v) {
  return ((v & 0x0F0F0F0Fu) << 4) | ((v >> 4) & 0x0F0F0F0Fu);
}

__global__ void retile_kernel(const uint8_t* __restrict__ path, int64_t ps,
                              const uint8_t* __restrict__ member, int64_t ms,
                              int64_t n, int64_t d, int bits, int64_t T, int64_t G,
                              uint32_t* __restrict__ out_path, uint32_t* __restrict__ out_member) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= T * G * kTileRows) return;
  const int r = (int)(idx & 15);
  const int64_t tg = idx >> 4;
  const int64_t g = tg % G, t = tg / G;
  const int64_t row = t * kTileRows + r;
  uint32_t h[2] = {0, 0};     // path bits of the two halves
  uint32_t mlo[4] = {0, 0, 0, 0};  // 2-bit member fields per 16-column group
  uint32_t m1[4] = {0, 0, 0, 0};   // 1-bit member fields per 16-column group
  if (row < n) {
    const uint8_t* prow = path + row * ps;
    const uint8_t* mrow = member ? member + row * ms : nullptr;
    for (int c = 0; c < kSegCols; ++c) {
      const int64_t col = g * kSegCols + c;
      if (col >= d) break;
      h[c >> 5] |= read_bits_le(prow, ps, col, 1) << (c & 31);
      if (bits > 1) {
        const uint32_t mv = read_bits_le(mrow, ms, col * (bits - 1), bits - 1);
        const int grp = c >> 4, j = c & 15;
        if (bits == 2) {
          m1[grp] |= (mv & 1u) << j;
        } else {
          mlo[grp] |= (mv & 3u) << (2 * j);
          if (bits == 4) m1[grp] |= ((mv >> 2) & 1u) << j;
        }
      }
    }
  }
  out_path[idx * 2] = interleave16(h[0] & 0xFFFFu, h[1] & 0xFFFFu);
  out_path[idx * 2 + 1] = interleave16(h[0] >> 16, h[1] >> 16);
  const int mw = member_words(bits);
  uint32_t* mo = out_member + idx * mw;
  // column groups: 0 = first half x=0, 1 = first half x=1, 2 = second half x=0, 3 = second half x=1;
  // 2-bit member words are stored with the two nibbles of every byte swapped
  // (the decoder's index formation pairs them with subset nibbles in one op)
  if (bits == 3 || bits == 4) {
    mo[0] = nibble_swap(mlo[0]); mo[1] = nibble_swap(mlo[2]);
    mo[2] = nibble_swap(mlo[1]); mo[3] = nibble_swap(mlo[3]);
  }
  if (bits == 2) {
    mo[0] = pair_interleave16(m1[0], m1[2]);
    mo[1] = pair_interleave16(m1[1], m1[3]);
  } else if (bits == 4) {
    mo[4] = high_member_word(m1[0], m1[2]);
    mo[5] = high_member_word(m1[1], m1[3]);
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
}  // namespace tp

using namespace tp;

extern "C" int tp_tiled_layout(int64_t n, int64_t d, int bits, int64_t* tiles, int64_t* segments,
                               int64_t* path_bytes, int64_t* member_bytes, int64_t* z_cols) {
  Geom g;
  int st = tiled_geom(n, d, bits, &g);
  if (st) return st;
  if (tiles) *tiles = g.T;
  if (segments) *segments = g.G;
  if (path_bytes) *path_bytes = g.path_words * 4;
  if (member_bytes) *member_bytes = g.member_words * 4;
  if (z_cols) *z_cols = g.G * kSegCols;
  return TP_OK;
}

extern "C" int tp_retile(const uint8_t* path, int64_t path_stride, const uint8_t* member,
                         int64_t member_stride, int64_t n, int64_t d, int bits,
                         uint8_t* path_tiled, uint8_t* member_tiled, void* stream) {
  Geom g;
  int st = tiled_geom(n, d, bits, &g);
  if (st) return st;
  if (!path || !member || !path_tiled || !member_tiled) return TP_ERR_NULL_POINTER;
  if (path_stride < (d + 7) / 8 || member_stride < (d * (bits - 1) + 7) / 8) return TP_ERR_BAD_DIMS;
  if (((uintptr_t)path_tiled | (uintptr_t)member_tiled) & 15) return TP_ERR_MISALIGNED;
  const int64_t threads = g.T * g.G * kTileRows;
  hipLaunchKernelGGL(retile_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, path, path_stride, member, member_stride, n, d, bits,
                     g.T, g.G, reinterpret_cast<uint32_t*>(path_tiled),
                     reinterpret_cast<uint32_t*>(member_tiled));
  return launch_status();
}

extern "C" int64_t tp_gemv_workspace_bytes(int64_t n, int64_t batch) {
  // (the tiled layout holds at most 2^26 row tiles)
  if (n <= 0 || n > ((int64_t)1 << 30) || batch <= 0 || batch > 32) return 0;
  const int64_t T = (n + kTileRows - 1) / kTileRows;
  const int64_t nbt = batch <= 16 ? 1 : 2;
  // split-K sums + counters of the batch 5..32 kernels, or the K-split
  // one-pass kernel's part slices + counters, whichever is larger
  return std::max<int64_t>(T * kTileRows * 16 * nbt * 4 + T * 4, linear_ksplit_bytes(T));
}

extern "C" int tp_decode_tiled(const uint8_t* path_tiled, const uint8_t* member_tiled,
                               const uint16_t* scales, const uint16_t* codebook,
                               int64_t n, int64_t d, int bits, int n_states,
                               uint16_t* w_out, int64_t out_stride, void* stream) {
  Geom g;
  int st = tiled_geom(n, d, bits, &g);
  if (st) return st;
  if (!path_tiled || !member_tiled || !scales || !codebook || !w_out) return TP_ERR_NULL_POINTER;
  if (out_stride < d) return TP_ERR_BAD_DIMS;
  const int64_t units = g.T * g.G4;
  dim3 grid((unsigned)((units + 3) / 4)), block(256);
  hipStream_t s = (hipStream_t)stream;
  const uint32_t* p = reinterpret_cast<const uint32_t*>(path_tiled);
  const uint32_t* m = reinterpret_cast<const uint32_t*>(member_tiled);
#define TP_DEC(KB, NS)                                                                            \
  hipLaunchKernelGGL((tiled_decode_kernel<KB, NS>), grid, block, 0, s, p, m, scales, codebook,  \
                     (int)n, (int)d, (int)g.T, (int)g.G, (int)g.G4, w_out, out_stride)
  switch (bits * 100 + n_states) {
    case 204: TP_DEC(2, 4); break;
    case 208: TP_DEC(2, 8); break;
    case 216: TP_DEC(2, 16); break;
    case 264: TP_DEC(2, 64); break;
    case 304: TP_DEC(3, 4); break;
    case 308: TP_DEC(3, 8); break;
    case 316: TP_DEC(3, 16); break;
    case 364: TP_DEC(3, 64); break;
    case 404: TP_DEC(4, 4); break;
    case 408: TP_DEC(4, 8); break;
    case 416: TP_DEC(4, 16); break;
    case 464: TP_DEC(4, 64); break;
    default: return TP_ERR_UNSUPPORTED_STATES;
  }
#undef TP_DEC
  return launch_status();
}

namespace tp {

// Dynamic LDS (z staging); the 64 KiB pair table is static.
constexpr size_t gemv_lds_bytes(int nbt) {
  return (size_t)16 * nbt * kZCols * 2;
}

template <int KB, int NS, int NBT, bool ROT>
void launch_gemv(const GemvArgs& a, int grid, hipStream_t s) {
  hipLaunchKernelGGL((tcq_gemv_tiled_kernel<KB, NS, NBT, ROT>), dim3(grid), dim3(kGroupThreads),
                     gemv_lds_bytes(NBT), s, a);
}

template <int KB, int NS>
void launch_gemv_kb(const GemvArgs& a, int grid, int nbt, bool rot, hipStream_t s) {
  if (nbt == 1) {
    rot ? launch_gemv<KB, NS, 1, true>(a, grid, s) : launch_gemv<KB, NS, 1, false>(a, grid, s);
  } else {
    rot ? launch_gemv<KB, NS, 2, true>(a, grid, s) : launch_gemv<KB, NS, 2, false>(a, grid, s);
  }
}

// clear_ws: the caller's workspaces may hold anything (the no-allocation
// entry point's shared array): each launch that uses one is preceded by a
// fill of the bytes it uses.  Otherwise workspaces are zero between calls,
// which every kernel restores.  A workspace too small for the split-K kernel
// is an error only when that kernel is the one that runs.
int gemv_tiled_group(const TiledLinearArgs* ls, int n_lin, int64_t batch, const uint16_t* codebook,
                     int bits, int n_states, void* stream, bool clear_ws) {
  if (n_lin < 1 || n_lin > kMaxInlineLinears) return TP_ERR_BAD_DIMS;
  if (!codebook) return TP_ERR_NULL_POINTER;
  if (bits < 2 || bits > 4) return TP_ERR_UNSUPPORTED_BITS;
  if (batch < 1 || batch > 32) return TP_ERR_BAD_DIMS;
  const int nbt = batch <= 16 ? 1 : 2;
  const bool rot = ls[0].rot_scale != nullptr;
  GemvArgs a;
  a.n_lin = n_lin;
  a.batch = (int)batch;
  a.codebook = codebook;
  int64_t units_total = 0;
  for (int i = 0; i < n_lin; ++i) {
    Geom g;
    int st = tiled_geom(ls[i].n, ls[i].d, bits, &g);
    if (st) return st;
    if ((ls[i].rot_scale != nullptr) != rot) return TP_ERR_BAD_LAYOUT;
    units_total += g.T * g.G4;
  }
  const int cus = device_cu_count();
  const int64_t max_waves = (int64_t)cus * 2 * kWavesPerGroup;
  int64_t kg = (units_total + max_waves - 1) / max_waves;
  if (kg < 1) kg = 1;
  if (kg > kMaxUnitsPerBlock) kg = kMaxUnitsPerBlock;
  int64_t total_blocks = 0;
  int ws_status = TP_OK;           // the split-K kernel's workspace check, reported if it runs
  int64_t ws_need[kMaxInlineLinears] = {0, 0, 0, 0};
  for (int i = 0; i < n_lin; ++i) {
    const TiledLinearArgs& l = ls[i];
    if (!l.path_tiled || !l.member_tiled || !l.x || !l.scales || !l.y) return TP_ERR_NULL_POINTER;
    Geom g;
    tiled_geom(l.n, l.d, bits, &g);
    if (l.ldy < l.n) return TP_ERR_BAD_DIMS;
    if (((uintptr_t)l.path_tiled & 15) || ((uintptr_t)l.member_tiled & 15)) return TP_ERR_MISALIGNED;
    LinearDesc& L = a.lin[i];
    if (rot) {
      const int64_t hb = l.block;
      if (hb < 1 || (hb & (hb - 1)) || l.d % hb || hb > 16384) return TP_ERR_BAD_BLOCK;
      if (l.ldx < l.d || (l.ldx & 3) || (l.d & 3) || ((uintptr_t)l.x & 7) || ((uintptr_t)l.rot_scale & 7))
        return TP_ERR_MISALIGNED;
      L.hb = (int32_t)hb;
      L.hdiv = (float)__builtin_sqrt((double)hb);
    } else {
      if (l.ldx < g.G * kSegCols || (l.ldx & 7) || ((uintptr_t)l.x & 15)) return TP_ERR_BAD_DIMS;
      L.hb = 1;
      L.hdiv = 1.f;
    }
    const int64_t kgl = kg < g.G4 ? kg : g.G4;
    const int64_t nkb = (g.G4 + kgl - 1) / kgl;
    const int64_t blocks = ((g.T + kWavesPerGroup - 1) / kWavesPerGroup) * nkb;
    L.path = reinterpret_cast<const uint32_t*>(l.path_tiled);
    L.member = reinterpret_cast<const uint32_t*>(l.member_tiled);
    L.x = l.x;
    L.rs = l.rot_scale;
    L.scales = l.scales;
    L.bias = l.bias;
    L.y = l.y;
    L.n = (int32_t)l.n;
    L.d = (int32_t)l.d;
    L.T = (int32_t)g.T;
    L.G = (int32_t)g.G;
    L.G4 = (int32_t)g.G4;
    L.ldx = (int32_t)l.ldx;
    L.ldy = (int32_t)l.ldy;
    L.kg = (int32_t)kgl;
    L.blocks = (int32_t)blocks;
    if (nkb > 1) {
      const int64_t need = g.T * kTileRows * 16 * nbt * 4 + g.T * 4;
      if (!l.workspace || l.workspace_bytes < need) {
        if (!ws_status) ws_status = TP_ERR_WORKSPACE;
      } else if ((uintptr_t)l.workspace & 15) {
        if (!ws_status) ws_status = TP_ERR_MISALIGNED;
      }
      ws_need[i] = need;
      L.ws = reinterpret_cast<float*>(l.workspace);
      L.cnt = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(l.workspace) + g.T * kTileRows * 16 * nbt * 4);
    } else {
      L.ws = nullptr;
      L.cnt = nullptr;
    }
    total_blocks += blocks;
  }
  for (int i = n_lin; i < kMaxInlineLinears; ++i) a.lin[i] = a.lin[0];
  if (total_blocks > INT32_MAX) return TP_ERR_BAD_DIMS;
  // Batch <= 8 runs the one-pass kernel (tp_linear.hip) when it applies.
  const int fast = linear_forward_fast(ls, n_lin, batch, codebook, bits, n_states, (hipStream_t)stream, clear_ws);
  if (fast != kLinearNotHandled) return fast;
  // Batch 9..32: 16-tile blocks through LDS (tp_stack.hip), on rotated
  // activations or rotating them in the launch (blocks <= 512).
  if (batch > 8) {
    bool wide = true;
    for (int i = 0; i < n_lin && rot; ++i)
      wide = wide && a.lin[i].hb <= kZCols && a.lin[i].d % 8 == 0 && a.lin[i].ldx % 8 == 0 &&
             !((uintptr_t)a.lin[i].x & 15) && !((uintptr_t)a.lin[i].rs & 15);
    if (wide) {
      for (int i = 0; i < n_lin; ++i) {
        if (clear_ws && ls[i].workspace && !((uintptr_t)ls[i].workspace & 15)) {
          // (the bytes the wide kernel uses when the workspace holds them)
          const int64_t wneed = (int64_t)a.lin[i].T * kTileRows * 16 * nbt * 4 + (int64_t)a.lin[i].T * 4;
          if (ls[i].workspace_bytes >= wneed) {
            const int zst = zero_device_bytes(ls[i].workspace, wneed, (hipStream_t)stream);
            if (zst) return zst;
          }
        }
        const int st = linear_forward_wide(a.lin[i], rot ? nullptr : ls[i].x, ls[i].ldx, batch, codebook, bits,
                                           n_states, ls[i].workspace, ls[i].workspace_bytes, (hipStream_t)stream);
        if (st) return st;
      }
      return TP_OK;
    }
  }
  if (ws_status) return ws_status;
  if (clear_ws) {
    for (int i = 0; i < n_lin; ++i) {
      if (!ws_need[i]) continue;
      const int zst = zero_device_bytes(ls[i].workspace, ws_need[i], (hipStream_t)stream);
      if (zst) return zst;
    }
  }
  a.total_blocks = (int32_t)total_blocks;
  const int wg_per_cu = nbt == 1 ? 2 : 1;
  int grid = (int)(total_blocks < (int64_t)cus * wg_per_cu ? total_blocks : (int64_t)cus * wg_per_cu);
  hipStream_t s = (hipStream_t)stream;
  switch (bits * 100 + n_states) {
    case 204: launch_gemv_kb<2, 4>(a, grid, nbt, rot, s); break;
    case 208: launch_gemv_kb<2, 8>(a, grid, nbt, rot, s); break;
    case 216: launch_gemv_kb<2, 16>(a, grid, nbt, rot, s); break;
    case 264: launch_gemv_kb<2, 64>(a, grid, nbt, rot, s); break;
    case 304: launch_gemv_kb<3, 4>(a, grid, nbt, rot, s); break;
    case 308: launch_gemv_kb<3, 8>(a, grid, nbt, rot, s); break;
    case 316: launch_gemv_kb<3, 16>(a, grid, nbt, rot, s); break;
    case 364: launch_gemv_kb<3, 64>(a, grid, nbt, rot, s); break;
    case 404: launch_gemv_kb<4, 4>(a, grid, nbt, rot, s); break;
    case 408: launch_gemv_kb<4, 8>(a, grid, nbt, rot, s); break;
    case 416: launch_gemv_kb<4, 16>(a, grid, nbt, rot, s); break;
    case 464: launch_gemv_kb<4, 64>(a, grid, nbt, rot, s); break;
    default: return TP_ERR_UNSUPPORTED_STATES;
  }
  return launch_status();
}

}  // namespace tp

extern "C" int tp_tcq_gemv_tiled(const uint16_t* z, int64_t ldz, int64_t batch,
                                 const uint8_t* path_tiled, const uint8_t* member_tiled,
                                 const uint16_t* scales, const uint16_t* codebook, const uint16_t* bias,
                                 int64_t n, int64_t d, int bits, int n_states,
                                 uint16_t* y, int64_t ldy, void* workspace, int64_t workspace_bytes,
                                 void* stream) {
  TiledLinearArgs l{path_tiled, member_tiled, z, ldz, nullptr, 0, scales, bias, y, ldy, n, d,
                    workspace, workspace_bytes};
  return gemv_tiled_group(&l, 1, batch, codebook, bits, n_states, stream, false);
}

extern "C" int tp_packed_linear_forward(const uint16_t* x, int64_t ldx, int64_t batch,
                                        const uint16_t* rot_scale, int64_t block,
                                        const uint8_t* path_tiled, const uint8_t* member_tiled,
                                        const uint16_t* scales, const uint16_t* codebook,
                                        const uint16_t* bias, int64_t n, int64_t d, int bits,
                                        int n_states, uint16_t* y, int64_t ldy, void* workspace,
                                        int64_t workspace_bytes, void* stream) {
  if (!rot_scale) return TP_ERR_NULL_POINTER;
  TiledLinearArgs l{path_tiled, member_tiled, x, ldx, rot_scale, block, scales, bias, y, ldy, n, d,
                    workspace, workspace_bytes};
  return gemv_tiled_group(&l, 1, batch, codebook, bits, n_states, stream, false);
}

namespace tp {
int packed_linear_forward_cleared(const uint16_t* x, int64_t ldx, int64_t batch, const uint16_t* rot_scale,
                                  int64_t block, const uint8_t* path_tiled, const uint8_t* member_tiled,
                                  const uint16_t* scales, const uint16_t* codebook, const uint16_t* bias, int64_t n,
                                  int64_t d, int bits, int n_states, uint16_t* y, int64_t ldy, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
  if (!rot_scale) return TP_ERR_NULL_POINTER;
  TiledLinearArgs l{path_tiled, member_tiled, x, ldx, rot_scale, block, scales, bias, y, ldy, n, d,
                    workspace, workspace_bytes};
  return gemv_tiled_group(&l, 1, batch, codebook, bits, n_states, stream, true);
}
}  // namespace tp

extern "C" int tp_packed_linear_forward_group(int n_linears, const uint16_t* x, int64_t ldx,
                                              int64_t batch, const uint16_t* const* rot_scales,
                                              const int64_t* blocks, const uint8_t* const* path_tiled,
                                              const uint8_t* const* member_tiled,
                                              const uint16_t* const* scales, const uint16_t* codebook,
                                              const uint16_t* const* biases, const int64_t* ns,
                                              int64_t d, int bits, int n_states, uint16_t* const* ys,
                                              const int64_t* ldys, void* const* workspaces,
                                              const int64_t* workspace_bytes, void* stream) {
  if (n_linears < 1 || n_linears > kMaxInlineLinears) return TP_ERR_BAD_DIMS;
  if (!rot_scales || !blocks || !path_tiled || !member_tiled || !scales || !ns || !ys || !ldys ||
      !workspaces || !workspace_bytes)
    return TP_ERR_NULL_POINTER;
  TiledLinearArgs ls[kMaxInlineLinears];
  for (int i = 0; i < n_linears; ++i) {
    if (!rot_scales[i]) return TP_ERR_NULL_POINTER;
    ls[i] = TiledLinearArgs{path_tiled[i], member_tiled[i], x, ldx, rot_scales[i], blocks[i],
                            scales[i], biases ? biases[i] : nullptr, ys[i], ldys[i], ns[i], d,
                            workspaces[i], workspace_bytes[i]};
  }
  return gemv_tiled_group(ls, n_linears, batch, codebook, bits, n_states, stream, false);
}
