// One persistent launch for every packed linear of a decode step.
//
// The reference runs a decode step as one graph node pair per projection
// (turbopress/runtime.py:312-316 inside the HF decoder, replayed by
// scripts/graph_decode_bench.py:103-115).  On MI355X a kernel launch inside a
// graph costs ~1.5 us and a 9.4 MB GEMV cannot reach HBM speed before its
// latency chain ends, so here one launch streams the whole list of linears:
//
//   * work = "blocks" of 8 row tiles x the full K range of one linear, handed
//     to persistent workgroups by an atomic ticket (self-resetting), in a
//     schedule stored in the plan (largest K first when unordered, so the
//     launch does not end on a long block);
//   * full-K blocks need no split-K reduction: each wave writes its 16 rows;
//   * optional phase ordering: linears carry a phase index and, when
//     `ordered` is set, a block of phase p starts only after every block of
//     phase p-1 has finished (bounded wait; on timeout the plan's error flag
//     is set and the block proceeds, so the kernel always terminates).
//
// A run is two kernels:
//   1. tcq_stack_rotate_kernel: z = blockFWHT(x * rot_scale) / sqrt(hb) of
//      every linear into the plan's z buffer (fp16, zero past d) -- a few
//      MB at batch 1, read back from L2/MALL;
//   2. batch <= 4 (the decode case): tcq_stack_slot_kernel: a wave streams
//      its tile's path/member words and z with buffer loads, three units
//      ahead, and never synchronises with the other waves inside a block.
//      Only `batch` of the 16 MFMA B columns carry data, so the columns are
//      split into 16/SB "slots" of SB batch rows: one 16-byte z load per
//      lane feeds 16/SB MFMAs (MFMA i reads its activations from slot
//      i % (16/SB) and accumulates into its own accumulator); the valid
//      column of each accumulator is summed across slots once per block.
//      The LDS then only serves the codebook pair table, whose lookups bound
//      the kernel's issue rate.
//      Batch 5..32: tcq_stack_wide_kernel: 16-wave workgroups stage the
//      rotated activations through LDS in 512-column chunks (double
//      buffered) and every wave reads them as MFMA B operands.
#include "tp_tiled_common.h"
#include "tp_slot.h"
#include "tp_rotate_tile.h"

#include <algorithm>
#include <mutex>
#include <unordered_map>
#include <type_traits>
#include <vector>

namespace tp {

constexpr int kStackMaxPhases = 4096;
// Schedule entries are int32 values (linear << kStackBlockBits) | block: a
// plan holds at most 2^16 linears of at most 2^14 blocks each (2M rows), so
// every entry stays positive.
constexpr int kStackBlockBits = 14;
constexpr int kStackMaxLinears = 1 << 16;
static_assert(((int64_t)kStackMaxLinears << kStackBlockBits) - 1 <= INT32_MAX,
              "schedule entries must fit a positive int32");
// Batches up to this use the slot kernel (4 batch rows per slot); larger ones
// the wide kernel, which at batch 8 measured 371 us per Qwen3-4B step
// against 475 us for 2 slots of 8 rows (whose z registers leave room for only
// one unit of loads in flight), and at batch 5 about the same.
constexpr int kSlotMaxBatch = 4;

// Plan layout (device memory):
//   [0, 64)             StackCounters  -- written by the kernels (atomics)
//   [64, ...)           StackInfo, RotItem[n_rot] (at the fixed offset
//                       kRotItems), LinearDesc[n_lin], prefix[n_lin+1],
//                       lphase[n_lin], pblocks[n_phases], sched_ordered[total],
//                       sched_unordered[total], wide schedules, ptiles[n_phases],
//                       ord_blocks[<= 8 total]  -- read-only
//   [pdone, ...)        pdone[n_phases] -- written by the kernel (atomics)
//   [zbuf, ...)         rotated activations
// The read-only part is passed as a separate const __restrict__ argument so
// its loads go through the scalar cache into SGPRs.
struct StackCounters {
  uint32_t ticket;   // next block index (reset to 0 by the last workgroup out)
  uint32_t exited;   // workgroups past the loop (reset likewise)
  uint32_t error;    // 1: a phase wait timed out; 2: launched for fewer batch rows than the plan
  uint32_t gen;      // ordered kernel: launches finished (phase counters count on across launches)
  uint32_t reserved[12];
};

struct StackInfo {
  int32_t n_lin;
  int32_t total_blocks;
  int32_t n_phases;
  int32_t batch;
  int32_t n_rot;          // rotation tiles (see rot_tiles) when the plan has a z buffer
  int32_t min_g4;         // shortest K of the plan in 256-column units
  int64_t zbuf_bytes;
  int32_t total_wide;     // wide blocks (16 tiles x full K) of the batch 5..32 kernel
  int32_t total_k;        // blocks of the ordered kernel (tile groups with K split across the waves)
  int32_t n_rot_packed;   // the first n_rot rotation tiles: packed tiles (blocks <= 4096); the rest above 4096
};

// One rotation item: a 4096-column tile, as a packed tile or one batch row's
// tile of a block above 4096 (see the rotation kernels).
struct RotItem {
  const uint16_t* x;    // input row 0 (packed) / the tile's input row
  const uint16_t* rs;   // rot_scale [d]
  uint16_t* z;          // z row 0 (packed) / the tile's z row
  int32_t k;            // packed: first block of the tile (row-major over batch rows); else tile index along d
  int32_t d;
  int32_t hb;
  int32_t zld;          // z columns per batch row
  float hdiv;           // fp32(sqrt(hb))
  int32_t ldx;          // packed: input row stride (elements)
  int32_t nblk;         // packed: blocks per batch row (d / hb)
  int32_t nbt;          // packed: blocks of the linear (batch * nblk)
  int32_t logh;         // log2(hb)
  float hrecip;         // fp32(1 / hdiv), correctly rounded
};
static_assert(sizeof(RotItem) == 64, "one 16-dword scalar load per rotation tile");

// One block of the ordered kernel: row tiles [t0, t0 + nt) of linear li.
struct OrdBlockDesc {
  int32_t li, t0, nt, reserved;
};
static_assert(sizeof(OrdBlockDesc) == 16, "one 4-dword scalar load per block");

struct StackLayout {
  size_t rot_items, lin, prefix, lphase, pblocks, sched_o, sched_u, sched_wo, sched_wu, ptiles, oblk, pdone,
      odone, zbuf, total;
};

// Ordered kernel: every phase counter is kept in kOrdReplicas copies on
// separate 128-byte lines (each workgroup adds its tiles to all of them and
// polls one), so that hundreds of waiting workgroups do not all poll one line.
constexpr int kOrdReplicas = 16;
constexpr int kOrdLineWords = 32;

constexpr size_t kStackRO = sizeof(StackCounters);
constexpr size_t kRotItems = (kStackRO + sizeof(StackInfo) + 63) & ~(size_t)63;  // fixed offset

// Reads of the plan's read-only part through the constant address space
// (TP_CONST): the plan does not change during a launch.
template <typename T>
__device__ __forceinline__ const TP_CONST T& cread(const T* p) {
  return *(const TP_CONST T*)p;
}

__host__ __device__ inline StackLayout stack_layout(int n_lin, int n_phases, int total_blocks, int n_rot,
                                                    int64_t zbuf_bytes) {
  StackLayout p;
  size_t o = kRotItems;
  p.rot_items = o;
  o += sizeof(RotItem) * (size_t)n_rot;
  p.lin = o;
  o += sizeof(LinearDesc) * (size_t)n_lin;
  p.prefix = o;
  o += sizeof(int32_t) * (size_t)(n_lin + 1);
  p.lphase = o;
  o += sizeof(int32_t) * (size_t)n_lin;
  p.pblocks = o;
  o += sizeof(int32_t) * (size_t)n_phases;
  p.sched_o = o;
  o += sizeof(int32_t) * (size_t)total_blocks;
  p.sched_u = o;
  o += sizeof(int32_t) * (size_t)total_blocks;
  p.sched_wo = o;  // wide schedules: at most one entry per 8-tile block
  o += sizeof(int32_t) * (size_t)total_blocks;
  p.sched_wu = o;
  o += sizeof(int32_t) * (size_t)total_blocks;
  p.ptiles = o;
  o += sizeof(int32_t) * (size_t)n_phases;
  p.oblk = o;  // ordered kernel: at most one block per row tile (8 per 8-tile block)
  o += sizeof(OrdBlockDesc) * (size_t)total_blocks * 8;
  o = (o + 63) & ~(size_t)63;
  p.pdone = o;
  o += sizeof(uint32_t) * (size_t)n_phases;
  o = (o + 127) & ~(size_t)127;
  p.odone = o;
  o += sizeof(uint32_t) * (size_t)n_phases * kOrdReplicas * kOrdLineWords;
  o = (o + 255) & ~(size_t)255;
  p.zbuf = o;
  o += (size_t)zbuf_bytes;
  p.total = (o + 255) & ~(size_t)255;
  return p;
}

struct StackRO {  // views into the read-only part
  const StackInfo* info;
  const LinearDesc* lin;
  const int32_t* prefix;   // [n_lin + 1] first block of each linear
  const int32_t* lphase;   // [n_lin]
  const int32_t* pblocks;  // [n_phases] blocks per phase
  const int32_t* sched_o;  // [total] (linear << kStackBlockBits) | block, phase order
  const int32_t* sched_u;  // [total] same blocks, longest K first
  const int32_t* sched_wo; // [total_wide] (linear << kStackBlockBits) | wide block, phase order
  const int32_t* sched_wu; // [total_wide] same, longest K first
  const int32_t* ptiles;   // [n_phases] row tiles per phase
  const OrdBlockDesc* oblk;  // [total_k] ordered-kernel blocks, phase order
  size_t pdone;            // byte offset of pdone from the plan start
  size_t odone;            // byte offset of the ordered kernel's replicated phase counters
  size_t zbuf;             // byte offset of the z buffer from the plan start
};

// `ro` points at plan + kStackRO.
__device__ inline StackRO stack_ro(const char* __restrict__ ro) {
  const StackInfo* info = reinterpret_cast<const StackInfo*>(ro);
  const TP_CONST StackInfo& ci = cread(info);
  const StackLayout l = stack_layout(ci.n_lin, ci.n_phases, ci.total_blocks, ci.n_rot, ci.zbuf_bytes);
  StackRO v;
  v.info = info;
  v.lin = reinterpret_cast<const LinearDesc*>(ro + (l.lin - kStackRO));
  v.prefix = reinterpret_cast<const int32_t*>(ro + (l.prefix - kStackRO));
  v.lphase = reinterpret_cast<const int32_t*>(ro + (l.lphase - kStackRO));
  v.pblocks = reinterpret_cast<const int32_t*>(ro + (l.pblocks - kStackRO));
  v.sched_o = reinterpret_cast<const int32_t*>(ro + (l.sched_o - kStackRO));
  v.sched_u = reinterpret_cast<const int32_t*>(ro + (l.sched_u - kStackRO));
  v.sched_wo = reinterpret_cast<const int32_t*>(ro + (l.sched_wo - kStackRO));
  v.sched_wu = reinterpret_cast<const int32_t*>(ro + (l.sched_wu - kStackRO));
  v.ptiles = reinterpret_cast<const int32_t*>(ro + (l.ptiles - kStackRO));
  v.oblk = reinterpret_cast<const OrdBlockDesc*>(ro + (l.oblk - kStackRO));
  v.pdone = l.pdone;
  v.odone = l.odone;
  v.zbuf = l.zbuf;
  return v;
}

// Bounded wait of one thread until every block of phase ph - 1 has finished.
__device__ inline void wait_phase(const StackRO& P, uint32_t* pdone, StackCounters* C, int ph,
                                  int spin_limit) {
  const uint32_t need = (uint32_t)cread(P.pblocks + ph - 1);
  int spins = 0;
  while (__hip_atomic_load(&pdone[ph - 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < need) {
    if (++spins > spin_limit) {
      atomicExch(&C->error, 1u);
      break;
    }
    __builtin_amdgcn_s_sleep(8);
  }
}

// ---------------------------------------------------------------------------
// 1. rotation of every linear's input into the plan's z buffer
// ---------------------------------------------------------------------------
// z = blockFWHT(x * rot_scale) / sqrt(hb) in fp32, rounded to fp16 once,
// with the stage order of the reference's transform (distance 1, 2, 4, ...
// then one division by sqrt(block)).
//
// Blocks of at most 4096 columns: a linear's (batch row, block) pairs,
// row-major, are packed densely into tiles of 4096 columns (4096 / hb
// blocks per tile, from as many batch rows as that takes), one 256-thread
// workgroup per tile, so that no work goes to columns past d (a
// 2560-column input at batch 32 is 20 tiles, not 32 tiles of 4096).
//
// The tile transform (thread layout, stages, division) is tp_rotate_tile.h;
// at 16 columns per thread this launch is bound by its VALU issue.
//
// Blocks above 4096 (H_hb = H_(hb/4096) (x) H_4096): one workgroup per
// 4096-column output tile of one batch row transforms each 4096-column
// sub-tile of its block, then runs the stages across sub-tiles (4096, 8192)
// in order.

// Rotation tiles of one linear: packed tiles of its batch * d columns when
// its block is at most 4096, else 4096-column tiles of each batch row.
__host__ __device__ inline int64_t rot_tiles(int64_t batch, int64_t d, int64_t hb) {
  return hb <= kRotTile ? (batch * d + kRotTile - 1) / kRotTile : batch * (d / kRotTile);
}

// One packed tile: load x * rot_scale, transform, divide, store z.
template <int LOGH, bool SWAP>
__device__ __forceinline__ void rot_packed_tile(const TP_CONST RotItem& L, int w, int m, int lane4, float* ex) {
  constexpr int HB = 1 << LOGH;
  const uint32_t nblk = (uint32_t)L.nblk, nbt = (uint32_t)L.nbt, ldx = (uint32_t)L.ldx;
  const uint32_t batch = nbt / nblk;
  const __amdgpu_buffer_rsrc_t xrs = buffer_rsrc(L.x, (uint32_t)((int64_t)(batch - 1) * ldx + L.d) * 2u);
  const __amdgpu_buffer_rsrc_t rrs = buffer_rsrc(L.rs, (uint32_t)L.d * 2u);
  // group g: tile columns 1024 w + 256 g + 4 m .. + 3, in block gb, batch
  // row b, columns col .. col + 3 of that row
  bool ok[4];
  uint32_t b[4], col[4];
  u32x2_t xw[4], rw[4];
  if constexpr (HB >= 256) {
    // the block and row are the wave's (scalar), the column inside the
    // block the lane's: one add per load.  A group past the tile's blocks
    // (the last tile) loads from byte offset 2^31 + 8 m (out of range:
    // zeros) and stores nothing.
    const uint32_t m8 = 8u * (uint32_t)m;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint32_t base = 1024u * (uint32_t)w + 256u * g;
      const uint32_t blk = (uint32_t)L.k + (base >> LOGH);
      const uint32_t row = (uint32_t)__builtin_amdgcn_readfirstlane((int)(blk / nblk));
      ok[g] = blk < nbt;
      b[g] = row;
      const uint32_t cu = (blk - row * nblk) * HB + (base & (HB - 1));  // (uniform)
      col[g] = cu + 4u * (uint32_t)m;
      const uint32_t xb = ok[g] ? (row * ldx + cu) * 2u : 0x80000000u;
      const uint32_t rb = ok[g] ? cu * 2u : 0x80000000u;
      uint32_t xo = xb + m8, ro = rb + m8;
      __asm__("" : "+v"(xo), "+v"(ro));
      xw[g] = __builtin_amdgcn_raw_buffer_load_b64(xrs, xo, 0, 0);
      rw[g] = __builtin_amdgcn_raw_buffer_load_b64(rrs, ro, 0, 0);
    }
  } else {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint32_t q = 1024u * (uint32_t)w + 256u * g + 4u * (uint32_t)m;
      const uint32_t gb = (uint32_t)L.k + (q >> LOGH);
      ok[g] = gb < nbt;
      b[g] = gb / nblk;
      col[g] = (gb - b[g] * nblk) * HB + (q & (HB - 1));
      xw[g] = load4h_words(xrs, ok[g] ? b[g] * ldx + col[g] : kOutOfRange / 2u);
      rw[g] = load4h_words(rrs, ok[g] ? col[g] : kOutOfRange / 2u);
    }
  }
  float v[kRotEPT];
  rot_products<(LOGH > 0)>(xw, rw, v);
  rot_stages<LOGH, SWAP>(v, w, m, lane4, ex);
  const float c = L.hdiv, r = L.hrecip;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    if (!ok[g]) continue;
    *(TP_GLOBAL u32x2_t*)(L.z + (size_t)b[g] * L.zld + col[g]) = rot_z4<LOGH>(v + 4 * g, c, r);
  }
}

// Packed tiles (items [0, n_rot_packed) of the plan), one workgroup per
// tile when the host knows the tile count (ONE_TILE: the descriptor is the
// first load, the x / rot_scale loads the second); otherwise a grid-stride
// loop bounded by the plan's count.  SWAP: see rot_lane_stage (the host
// takes it for launches of at most a few tiles per CU).
template <bool ONE_TILE, bool SWAP>
__global__ void __launch_bounds__(kRotThreads)
tcq_stack_rotate_kernel(const char* __restrict__ plan_ro) {
  __shared__ float ex[kRotTile];
  const int first = blockIdx.x;
  const int end = ONE_TILE ? first + 1 : cread(reinterpret_cast<const StackInfo*>(plan_ro)).n_rot_packed;
  const int step = ONE_TILE ? 1 : (int)gridDim.x;
  const RotItem* items = reinterpret_cast<const RotItem*>(plan_ro + (kRotItems - kStackRO));
  const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = (int)threadIdx.x & 63;
  const int m = rot_lane_index(lane), lane4 = 4 * lane;
  for (int item = first; item < end; item += step) {
    const TP_CONST RotItem& L = cread(items + item);
    // the descriptor's fields in one round trip
    __asm__ volatile("" ::"s"(L.x), "s"(L.rs), "s"(L.z), "s"(L.k), "s"(L.d), "s"(L.zld), "s"(L.hdiv),
                     "s"(L.ldx), "s"(L.nblk), "s"(L.nbt), "s"(L.logh), "s"(L.hrecip)
                     : "memory");
    switch (L.logh) {  // (uniform)
      case 0: rot_packed_tile<0, SWAP>(L, w, m, lane4, ex); break;
      case 1: rot_packed_tile<1, SWAP>(L, w, m, lane4, ex); break;
      case 2: rot_packed_tile<2, SWAP>(L, w, m, lane4, ex); break;
      case 3: rot_packed_tile<3, SWAP>(L, w, m, lane4, ex); break;
      case 4: rot_packed_tile<4, SWAP>(L, w, m, lane4, ex); break;
      case 5: rot_packed_tile<5, SWAP>(L, w, m, lane4, ex); break;
      case 6: rot_packed_tile<6, SWAP>(L, w, m, lane4, ex); break;
      case 7: rot_packed_tile<7, SWAP>(L, w, m, lane4, ex); break;
      case 8: rot_packed_tile<8, SWAP>(L, w, m, lane4, ex); break;
      case 9: rot_packed_tile<9, SWAP>(L, w, m, lane4, ex); break;
      case 10: rot_packed_tile<10, SWAP>(L, w, m, lane4, ex); break;
      case 11: rot_packed_tile<11, SWAP>(L, w, m, lane4, ex); break;
      case 12: rot_packed_tile<12, SWAP>(L, w, m, lane4, ex); break;
      default: break;
    }
  }
}

// Tiles of blocks above 4096 (items [n_rot_packed, n_rot) of the plan).
// H_hb = H_(hb/4096) (x) H_4096, stages in order of distance: every
// 4096-column sub-tile of the block through distances 1..2048, then
// distance 4096 (sub-tile pairs) and 8192 (pairs of pairs); sub-tile o of
// the result takes the signs of row o.
template <bool ONE_TILE, bool SWAP>
__global__ void __launch_bounds__(kRotThreads)
tcq_stack_rotate_big_kernel(const char* __restrict__ plan_ro) {
  __shared__ float ex[kRotTile];
  const TP_CONST StackInfo& ci = cread(reinterpret_cast<const StackInfo*>(plan_ro));
  const int base = ci.n_rot_packed;
  const int first = base + (int)blockIdx.x;
  const int end = ONE_TILE ? first + 1 : ci.n_rot;
  const int step = ONE_TILE ? 1 : (int)gridDim.x;
  const RotItem* items = reinterpret_cast<const RotItem*>(plan_ro + (kRotItems - kStackRO));
  const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = (int)threadIdx.x & 63;
  const int m = rot_lane_index(lane), lane4 = 4 * lane;
  for (int item = first; item < end; item += step) {
    const TP_CONST RotItem& L = cread(items + item);
    __asm__ volatile("" ::"s"(L.x), "s"(L.rs), "s"(L.z), "s"(L.k), "s"(L.d), "s"(L.hb), "s"(L.zld), "s"(L.hdiv),
                     "s"(L.hrecip)
                     : "memory");
    const int nsub = L.hb / kRotTile;        // 2 or 4
    const int o = L.k % nsub, k0 = L.k - o;  // this tile's sub-tile, the block's first
    const float s1 = (o & 1) ? -1.f : 1.f, s2 = (o & 2) ? -1.f : 1.f;
    const __amdgpu_buffer_rsrc_t xrs = buffer_rsrc(L.x, (uint32_t)L.d * 2u);
    const __amdgpu_buffer_rsrc_t rrs = buffer_rsrc(L.rs, (uint32_t)L.d * 2u);
    float v[kRotEPT], a[kRotEPT];
#pragma unroll 1
    for (int i = 0; i < nsub; ++i) {
      u32x2_t xw[4], rw[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint32_t off = (uint32_t)((k0 + i) * kRotTile + rot_col(w, m, 4 * g));
        xw[g] = load4h_words(xrs, off);
        rw[g] = load4h_words(rrs, off);
      }
      float t[kRotEPT];
      rot_products<true>(xw, rw, t);
      rot_stages<kRotMaxLogH, SWAP>(t, w, m, lane4, ex);
      if ((i & 1) == 0) {
#pragma unroll
        for (int e = 0; e < kRotEPT; ++e) a[e] = t[e];
      } else {
#pragma unroll
        for (int e = 0; e < kRotEPT; ++e) a[e] = __builtin_fmaf(s1, t[e], a[e]);  // distance 4096
        if (i == 1) {
#pragma unroll
          for (int e = 0; e < kRotEPT; ++e) v[e] = a[e];
        } else {
#pragma unroll
          for (int e = 0; e < kRotEPT; ++e) v[e] = __builtin_fmaf(s2, a[e], v[e]);  // distance 8192
        }
      }
    }
    // z = v / sqrt(hb) into the item's z row (hb > 4096 divides d: zld = d);
    // log2 hb is 13 or 14: the corrected quotient serves both
    const float c = L.hdiv, r = L.hrecip;
#pragma unroll
    for (int g = 0; g < 4; ++g)
      *(TP_GLOBAL u32x2_t*)(L.z + L.k * kRotTile + rot_col(w, m, 4 * g)) = rot_z4<1>(v + 4 * g, c, r);
  }
}

// ---------------------------------------------------------------------------
// 2. slot kernel (batch <= 4)
// ---------------------------------------------------------------------------

// Read-only state of one wave of the slot kernel.
struct SlotEnv {
  StackRO P;
  const int32_t* sched;
  const char* zbuf;
  StackCounters* C;
  uint32_t* pdone;
  const uint32_t* table;
  __amdgpu_buffer_rsrc_t zrs;   // the whole z buffer
  int total, batch, wave, lane, q, slot, bb, ordered, spin_limit, tid;
  uint32_t tbase;  // blocks [0, tbase) are assigned by workgroup index, the rest by ticket
  uint32_t laneoff, pv, mv;
};

// A block of the stream as one wave sees it (wave-uniform).
struct BlockInfo {
  int li;
  int t;    // row tile of this wave
  int G4;   // units along K; 0 when the ticket is past the end of the work
};

__device__ __forceinline__ BlockInfo stream_info(const SlotEnv& E, int blk) {
  BlockInfo b;
  const bool valid = blk < E.total;
  const int e = cread(E.sched + (valid ? blk : 0));
  b.li = __builtin_amdgcn_readfirstlane(e >> kStackBlockBits);
  b.t = (e & ((1 << kStackBlockBits) - 1)) * kWavesPerGroup + E.wave;
  b.G4 = valid ? cread(E.P.lin + b.li).G4 : 0;
  return b;
}

// Where the stream loads from: buffer descriptors of one block's tile of
// path/member words, the linear's z rows and this lane's z offsets.
template <int NZ>
struct LoadCtx {
  __amdgpu_buffer_rsrc_t prs, mrs;
  uint32_t zoff;       // byte offset of the linear's z rows in the z buffer
  uint32_t zv[NZ];     // lane offsets inside the z rows (per-lane)
  int G4;
};

template <int MW, int SB, int NZ>
__device__ __forceinline__ LoadCtx<NZ> stream_ctx(const SlotEnv& E, const BlockInfo& b) {
  constexpr int SLOTS = 16 / SB;
  const TP_CONST LinearDesc& L = cread(E.P.lin + b.li);
  const int tt = b.t < L.T ? b.t : 0;
  LoadCtx<NZ> c;
  const uint32_t unit_p = 4u * kTileRows * 8u, unit_m = 4u * kTileRows * MW * 4u;
  c.prs = buffer_rsrc(reinterpret_cast<const char*>(L.path) + (size_t)tt * L.G * (kTileRows * 2 * 4),
                      (uint32_t)L.G4 * unit_p);
  c.mrs = buffer_rsrc(reinterpret_cast<const char*>(L.member) + (size_t)tt * L.G * (kTileRows * MW * 4),
                      (uint32_t)L.G4 * unit_m);
  c.zoff = (uint32_t)(reinterpret_cast<const char*>(L.z) - E.zbuf);
  const uint32_t zld = (uint32_t)L.G4 * kChunkCols;
#pragma unroll
  for (int l = 0; l < NZ; ++l) {
    const int i = l * SLOTS + E.slot;  // the MFMA whose B column this lane supplies
    c.zv[l] = E.bb < E.batch ? ((uint32_t)E.bb * zld + (uint32_t)(E.q * kSegCols + mfma_col(i))) * 2u
                             : kOutOfRange;  // out of range: zeros, no memory traffic
  }
  c.G4 = b.G4;
  return c;
}

template <int MW, int NZ>
__device__ __forceinline__ UnitRegs<MW, NZ> stream_load(const SlotEnv& E, const LoadCtx<NZ>& c, int gu) {
  constexpr uint32_t unit_p = 4u * kTileRows * 8u;        // path bytes per unit
  constexpr uint32_t unit_m = 4u * kTileRows * MW * 4u;   // member bytes per unit
  constexpr uint32_t unit_z = kChunkCols * 2u;            // z bytes per unit and batch row
  UnitRegs<MW, NZ> g;
  // (at k=2 the unit index is pinned to a scalar register: left alone, the
  // compiler kept it in a vector one there and put both weight loads into
  // waterfall loops; at k=3 and 4 it stays scalar by itself, and the pin
  // would cost a VALU instruction per unit)
  const uint32_t ug = MW == 2 ? (uint32_t)__builtin_amdgcn_readfirstlane(gu) : (uint32_t)gu;
  g.X = __builtin_amdgcn_raw_buffer_load_b64(c.prs, E.pv, ug * unit_p, weight_policy(MW));
  g.M = MemberBuf<MW>::load(c.mrs, E.mv, ug * unit_m);
  // (uniform by construction; readfirstlane keeps it in a scalar register
  // when the compiler merges it with per-lane values)
  const uint32_t zs = (uint32_t)__builtin_amdgcn_readfirstlane((int)(c.zoff + (uint32_t)gu * unit_z));
#pragma unroll
  for (int l = 0; l < NZ; ++l) g.Z[l] = __builtin_amdgcn_raw_buffer_load_b128(E.zrs, c.zv[l], zs, 0);
  return g;
}

// Row scales of the lane's rows 4q..4q+3 of a block (range-checked: rows
// past n read 0 and are never written).
struct Scales4 { uint32_t v[4]; };
__device__ __forceinline__ Scales4 stream_scales(const SlotEnv& E, const BlockInfo& b) {
  const TP_CONST LinearDesc& L = cread(E.P.lin + b.li);
  const __amdgpu_buffer_rsrc_t srs = buffer_rsrc(L.scales, (uint32_t)L.n * 2u);
  const uint32_t off = (uint32_t)(b.t * kTileRows + 4 * E.q) * 2u;
  Scales4 s;
#pragma unroll
  for (int i = 0; i < 4; ++i) s.v[i] = __builtin_amdgcn_raw_buffer_load_b16(srs, off + 2u * i, 0, 0);
  return s;
}

__device__ __forceinline__ void stream_phase_wait(const SlotEnv& E, int li) {
  if (!E.ordered) return;
  const int ph = cread(E.P.lphase + li);
  if (ph > 0) {
    if (E.tid == 0) wait_phase(E.P, E.pdone, E.C, ph, E.spin_limit);
    __syncthreads();
  }
}

// The stream of one wave (see tcq_stack_slot_kernel) with D register sets.
// Blocks of the workgroup: cur (being decoded), nxt (known: its ticket was
// broadcast at the previous block end) and the one after (claimed by thread
// 0, published at the end of cur).  The load cursor runs D - 1 units ahead
// of the decoder, in cur or in nxt.
template <int KB, int NS, int SB, int D>
__device__ __forceinline__ void slot_stream(const SlotEnv& E, int blk0, int blk1, uint32_t pend, int* s_tk,
                                            uint32_t* table, const uint16_t* codebook) {
  constexpr int MW = member_words(KB);
  constexpr int SLOTS = 16 / SB;
  constexpr int NZ = 8 / SLOTS;
  // The first two schedule entries, then every field of their descriptors
  // that the stream's start reads, one round trip each (see the kernel);
  // stream_info and the rest read them again from the scalar cache.
  {
    const int e0 = cread(E.sched + (blk0 < E.total ? blk0 : 0));
    const int e1 = cread(E.sched + (blk1 < E.total ? blk1 : 0));
    __asm__ volatile("" ::"s"(e0), "s"(e1) : "memory");
    const TP_CONST LinearDesc& L0 = cread(E.P.lin + __builtin_amdgcn_readfirstlane(e0 >> kStackBlockBits));
    const TP_CONST LinearDesc& L1 = cread(E.P.lin + __builtin_amdgcn_readfirstlane(e1 >> kStackBlockBits));
    __asm__ volatile("" ::"s"(L0.path), "s"(L0.member), "s"(L0.scales), "s"(L0.z), "s"(L0.n), "s"(L0.T),
                     "s"(L0.G), "s"(L0.G4), "s"(L1.path), "s"(L1.member), "s"(L1.z), "s"(L1.T), "s"(L1.G),
                     "s"(L1.G4)
                     : "memory");
  }
  BlockInfo cur = stream_info(E, blk0);
  BlockInfo nxt = stream_info(E, blk1);
  if (cur.G4 == 0) return;
  LoadCtx<NZ> lc = stream_ctx<MW, SB, NZ>(E, cur);
  bool lnext = false;           // the load cursor is in nxt
  int lgu = 0;                  // next unit to load
  int pgu = 0;                  // next unit of cur to decode
  int bseq = 0;                 // blocks finished by this workgroup
  UnitRegs<MW, NZ> R[D];
  float4_t acc[SLOTS];
#pragma unroll
  for (int s = 0; s < SLOTS; ++s) acc[s] = float4_t{0.f, 0.f, 0.f, 0.f};
  uint32_t x1_last = 0;
  Scales4 sc = stream_scales(E, cur);
  stream_phase_wait(E, cur.li);

  // Load the cursor's unit into set k, then advance the cursor; at the end
  // of cur it moves into nxt, at the end of nxt (or of the work) it stays and
  // reloads its unit (in range, never decoded).
#define TP_STREAM_ISSUE(k)                                     \
  do {                                                         \
    R[k] = stream_load<MW, NZ>(E, lc, lgu);                    \
    if (lgu + 1 < lc.G4) {                                     \
      ++lgu;                                                   \
    } else if (!lnext && nxt.G4 > 0) {                         \
      lc = stream_ctx<MW, SB, NZ>(E, nxt);                     \
      lnext = true;                                            \
      lgu = 0;                                                 \
    }                                                          \
  } while (0)

#pragma unroll
  for (int k = 0; k < D - 1; ++k) TP_STREAM_ISSUE(k);
  // The pair table, built while the first units' loads are in flight: built
  // first, it held every first weight load ~2 us behind the launch's start.
  // The codebook comes through the scalar cache (codebook_lane_scalar).
  build_pair_table_lanes<KB>(table, codebook_lane_scalar<KB>(codebook, E.lane), E.tid, kGroupThreads);
  __syncthreads();

  for (;;) {
#pragma unroll
    for (int k = 0; k < D; ++k) {
      TP_STREAM_ISSUE((k + D - 1) % D);
      // Halo: word 1 of the previous segment comes from the lane 16 below
      // (K block q-1); lanes of K block 0 take the previous unit's last
      // segment (from lanes of K block 3, carried in x1_last); zero at a
      // row start (x1_last is cleared at every block end, not tested per
      // unit).
      const uint32_t provide = (E.q == 3) ? x1_last : R[k].X[1];
      slot_unit<KB, NS, SB, MW, NZ>(R[k], provide, E.lane, E.laneoff, E.table, acc);
      x1_last = R[k].X[1];
      if (++pgu == cur.G4) {
        x1_last = 0u;  // (the next block starts a row)
        // Block end: accumulator `slot` holds this lane's valid column; sum
        // the slots of each batch row, lanes of slot 0 write rows 4q..4q+3.
        const TP_CONST LinearDesc& L = cread(E.P.lin + cur.li);
        // the slot-0 lanes' column sums (DPP adds across the row)
        float4_t v = slot_column_sums<SLOTS, SB>(acc);
        // (the sums stay ahead of the store branch, where each DPP move folds
        // into its add; sunk into the branch, the moves stayed outside)
        __asm__ volatile("" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]));
        if (cur.t < L.T && E.slot == 0 && E.bb < E.batch) {
          const int row0 = cur.t * kTileRows + 4 * E.q;
          uint16_t* yr = L.y + (size_t)E.bb * L.ldy + row0;
          // Rows 4q..4q+3 in one 8-byte store when all four exist, there is
          // no bias and y's rows are 8-byte aligned (the same values as the
          // row-by-row stores; one address instead of four).
          const bool quad = !L.bias && ((reinterpret_cast<uintptr_t>(L.y) | ((uintptr_t)L.ldy << 1)) & 7u) == 0;
          if (quad && row0 + 4 <= L.n) {
            u32x2_t o;
            o.x = (uint32_t)f2h(v[0] * h2f((uint16_t)sc.v[0])) |
                  ((uint32_t)f2h(v[1] * h2f((uint16_t)sc.v[1])) << 16);
            o.y = (uint32_t)f2h(v[2] * h2f((uint16_t)sc.v[2])) |
                  ((uint32_t)f2h(v[3] * h2f((uint16_t)sc.v[3])) << 16);
            *(TP_GLOBAL u32x2_t*)yr = o;
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int row = row0 + i;
              if (row >= L.n) continue;
              uint16_t out = f2h(v[i] * h2f((uint16_t)sc.v[i]));
              if (L.bias) out = f2h(h2f(out) + h2f(gld(L.bias + row)));
              gst(yr + i, out);
            }
          }
        }
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) acc[s] = float4_t{0.f, 0.f, 0.f, 0.f};
        if (E.ordered) {
          __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
          __syncthreads();
          if (E.tid == 0) atomicAdd(&E.pdone[cread(E.P.lphase + cur.li)], 1u);
        }
        if (nxt.G4 == 0) return;
        // nxt becomes cur; the ticket claimed during this block names the
        // block after it (double-buffered slot: a slot is rewritten two
        // block ends later, after every wave has read it).
        if (E.tid == 0) s_tk[bseq & 1] = (int)pend;
        __syncthreads();
        const int blk = __builtin_amdgcn_readfirstlane(s_tk[bseq & 1]);
        ++bseq;
        if (E.tid == 0 && blk < E.total) pend = E.tbase + atomicAdd(&E.C->ticket, 1u);
        cur = nxt;
        nxt = stream_info(E, blk);
        lnext = false;  // the load cursor is in the new cur
        pgu = 0;
        sc = stream_scales(E, cur);
        stream_phase_wait(E, cur.li);
      }
    }
  }
#undef TP_STREAM_ISSUE
}

constexpr int kStreamDepth = 4;  // unit register sets of the stream (plans whose K >= 3 units)

// Persistent stream of units: the workgroup walks its blocks (tickets claimed
// two blocks ahead) and every wave streams its tile's units with D - 1 units
// of loads in flight, across block boundaries (the next block's first units
// load while the current block's last units are decoded).  With every block
// at least D - 1 units long (D is picked from the plan's shortest K), the
// load cursor never runs past the next block.  Every load is issued
// unconditionally (after the last block, an in-range unit is reloaded and
// never used), so the number of loads in flight is the same on every path
// and each wait covers the oldest register set only.
// What the host knows of a plan it initialised (lin_off == 0: nothing; the
// kernel then reads and checks the plan header).
struct PlanArgs {
  int64_t lin_off;    // byte offset of the LinearDesc array from plan_ro
  int64_t sched_off;  // byte offset of the launch's block schedule from plan_ro
  int32_t total;      // blocks of the plan
  int32_t batch;      // batch rows of the plan (<= SB)
};

template <int KB, int NS, int SB>
__global__ void __launch_bounds__(kGroupThreads) __attribute__((amdgpu_waves_per_eu(4)))
tcq_stack_slot_kernel(const char* __restrict__ plan_ro, char* __restrict__ plan_rw,
                      const uint16_t* __restrict__ codebook, int ordered, int spin_limit,
                      PlanArgs pa) {
  __shared__ __attribute__((aligned(16))) uint32_t table[kTableWords];
  __shared__ int s_tk[2];
  constexpr int MW = member_words(KB);
  // The scalar loads of the launch's start in as few dependent round trips
  // as their addresses allow: the kernel arguments, then the plan header,
  // then (in slot_stream) the first two schedule entries, then their
  // descriptors.  Left to the compiler, most fields waited for the one
  // before (~8 round trips, ~3 us at a launch's start, when every
  // workgroup asks for the same lines).  Each asm names the values to load
  // together; the memory clobber keeps later loads below it.
  __asm__ volatile("" ::"s"(plan_ro), "s"(plan_rw), "s"(codebook), "s"(ordered), "s"(spin_limit),
                   "s"(pa.lin_off), "s"(pa.sched_off), "s"(pa.total), "s"(pa.batch)
                   : "memory");
  {
    // (with the header, the codebook's first dword: its line is then in the
    // scalar cache when the pair table is built, after the first weight
    // loads -- fetched only then, it queued behind them, ~2 us)
    const TP_CONST StackInfo& ci = cread(reinterpret_cast<const StackInfo*>(plan_ro));
    __asm__ volatile("" ::"s"(ci.n_lin), "s"(ci.total_blocks), "s"(ci.n_phases), "s"(ci.batch), "s"(ci.n_rot),
                     "s"(ci.min_g4), "s"(ci.zbuf_bytes), "s"(cread(reinterpret_cast<const uint32_t*>(codebook)))
                     : "memory");
  }
  SlotEnv E;
  E.P = stack_ro(plan_ro);
  E.C = reinterpret_cast<StackCounters*>(plan_rw);
  if (pa.lin_off) {
    // A plan the host set up and checked: the first block's schedule and
    // descriptor loads do not wait for the plan header.
    E.P.lin = reinterpret_cast<const LinearDesc*>(plan_ro + pa.lin_off);
    E.sched = reinterpret_cast<const int32_t*>(plan_ro + pa.sched_off);
    E.total = pa.total;
    E.batch = pa.batch;
  } else {
    E.sched = ordered ? E.P.sched_o : E.P.sched_u;
    E.total = cread(E.P.info).total_blocks;
    E.batch = cread(E.P.info).batch;
    if (E.batch > SB || cread(E.P.info).n_rot <= 0) {  // not a plan for this kernel
      if (threadIdx.x == 0 && blockIdx.x == 0) atomicExch(&E.C->error, 2u);
      return;
    }
  }
  E.zbuf = plan_rw + E.P.zbuf;
  E.pdone = reinterpret_cast<uint32_t*>(plan_rw + E.P.pdone);
  E.table = table;
  E.ordered = ordered;
  E.spin_limit = spin_limit;
  E.tid = threadIdx.x;
  E.lane = E.tid & 63;
  E.wave = __builtin_amdgcn_readfirstlane(E.tid >> 6);
  const int r = E.lane & 15;
  E.q = E.lane >> 4;
  E.slot = r / SB;
  E.bb = r % SB;
  E.laneoff = lane_offsets<KB>(E.lane);
  E.pv = (uint32_t)(E.q * kTileRows + r) * 8u;        // path byte offset in a unit
  E.mv = (uint32_t)(E.q * kTileRows + r) * MW * 4u;   // member byte offset in a unit
  E.zrs = buffer_rsrc(plan_rw + E.P.zbuf, (uint32_t)cread(E.P.info).zbuf_bytes);

  // The first three blocks of every workgroup follow from its index: the
  // first weight loads wait for no ticket, and the first ticket atomics
  // happen at block ends, spread out in time, instead of all workgroups
  // hitting the counter at once.  Later blocks are claimed by ticket (offset
  // by the 3 * grid blocks handed out this way).
  E.tbase = 3u * gridDim.x;
  const int blk0 = (int)blockIdx.x;
  const int blk1 = (int)(blockIdx.x + gridDim.x);
  uint32_t pend = blockIdx.x + 2u * gridDim.x;  // thread 0: the block after blk1
  // Register sets: 4 for 4 z columns per lane set (SB = 4), 2 for SB = 8
  // (four z loads per unit); 2 when a block is shorter than the pipeline.
  constexpr int DMAX = SB <= 4 ? kStreamDepth : 2;
  if (cread(E.P.info).min_g4 >= DMAX - 1)
    slot_stream<KB, NS, SB, DMAX>(E, blk0, blk1, pend, s_tk, table, codebook);
  else
    slot_stream<KB, NS, SB, 2>(E, blk0, blk1, pend, s_tk, table, codebook);

  // The last workgroup out resets the counters for the next launch.
  if (E.tid == 0) {
    const uint32_t ex = atomicAdd(&E.C->exited, 1u);
    if (ex == gridDim.x - 1) {
      for (int p = 0; p < cread(E.P.info).n_phases; ++p) atomicExch(&E.pdone[p], 0u);
      atomicExch(&E.C->ticket, 0u);
      atomicExch(&E.C->exited, 0u);
    }
  }
}

// ---------------------------------------------------------------------------
// 2b. ordered kernel (batch <= 4, the decoder's phase order enforced)
// ---------------------------------------------------------------------------
// A linear of phase p may start only after every linear of phase p - 1 has
// finished.  Most phases hold far less work than the chip (one Qwen3-4B
// layer, in units of 16 rows x 256 columns: q/k/v 3840, o 2560, gate/up
// 12160, down 6080; 4096 waves), so a phase costs its latency chain: phase
// wait, decode, the sum over K, the y stores and the count.  The plan
// therefore cuts each phase into at most `grid` blocks where shapes allow
// (whole row tiles of one linear, balanced by units), so that a workgroup
// holds about one block per phase.  A block's units, tile-major, are split
// into 8 contiguous chunks, one per wave (a chunk spans at most 4 tiles); a
// wave loads the first units of its chunk, its halo word and the scales of
// the tiles it finishes BEFORE the phase wait, while the previous phase is
// still running, and streams the rest of the chunk through the same
// registers.  Per-tile partial sums go through LDS and are added in wave
// order (deterministic); wave w finishes tiles w, w + 8 and w + 16.  Blocks
// are handed out by index in phase order (block b to workgroup b % grid):
// every block a workgroup waits on was handed to a workgroup that reaches it
// first, so the waits always end.  The phase counters count finished row
// tiles.

// Tiles per block: a wave's chunk, ceil(nt * G4 / 8) <= 3 * G4 units, then
// spans at most kOrdSegs tiles; every wave finishes kOrdFinish of them.
constexpr int kOrdMaxTiles = 24;
constexpr int kOrdSegs = 4;
constexpr int kOrdFinish = kOrdMaxTiles / kWavesPerGroup;
static_assert(kOrdFinish * kWavesPerGroup == kOrdMaxTiles, "tiles finished per wave");

// Units of a wave's chunk held in registers at once (4 bits: the member
// words take the registers of the fourth).
__host__ __device__ constexpr int ord_max_units(int bits) { return bits == 4 ? 3 : 4; }

// Blocks of the ordered kernel for the linears [i0, i1) of one phase: at
// most `grid` where kOrdMaxTiles tiles per block allow, sized by units.
inline int64_t ord_phase_blocks(const LinearDesc* lin, int i0, int i1, int grid, OrdBlockDesc* out) {
  int64_t units = 0;
  for (int i = i0; i < i1; ++i) units += (int64_t)lin[i].T * lin[i].G4;
  // tiles per block of linear i for a target of tg units per block (and at
  // most 2^21 units per block, so that byte offsets stay 32-bit)
  auto tpb = [&](int i, int64_t tg) {
    const int64_t cap = std::max<int64_t>(1, std::min<int64_t>(kOrdMaxTiles, ((int64_t)1 << 21) / lin[i].G4));
    return (int)std::min<int64_t>(cap, std::max<int64_t>(1, tg / lin[i].G4));
  };
  auto count = [&](int64_t tg) {
    int64_t c = 0;
    for (int i = i0; i < i1; ++i) c += (lin[i].T + tpb(i, tg) - 1) / tpb(i, tg);
    return c;
  };
  auto capped = [&](int64_t tg) {
    for (int i = i0; i < i1; ++i)
      if (tpb(i, tg) < tpb(i, (int64_t)1 << 40)) return false;
    return true;
  };
  int64_t tg = std::max<int64_t>(1, (units + grid - 1) / grid);
  while (count(tg) > grid && !capped(tg)) tg += std::max<int64_t>(1, tg / 16);
  int64_t nb = 0;
  for (int i = i0; i < i1; ++i) {
    const int t = tpb(i, tg);
    for (int t0 = 0; t0 < lin[i].T; t0 += t) out[nb++] = {i, t0, std::min(t, lin[i].T - t0), 0};
  }
  return nb;
}

// Bounded wait of one thread until every row tile of phase ph - 1 has
// finished in this launch: replica r of the phase's counter has reached
// (gen + 1) * tiles (counters count on across launches, modulo 2^32).
__device__ inline void wait_phase_replica(const StackRO& P, const uint32_t* odone, StackCounters* C, int ph,
                                          uint32_t gen, int r, int spin_limit) {
  const uint32_t need = (gen + 1u) * (uint32_t)cread(P.ptiles + ph - 1);
  const uint32_t* ctr = odone + ((size_t)(ph - 1) * kOrdReplicas + r) * kOrdLineWords;
  int spins = 0;
  while ((int32_t)(__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - need) < 0) {
    if (++spins > spin_limit) {
      atomicExch(&C->error, 1u);
      break;
    }
    // (polls 512 cycles apart: 256 measured 1237 us per ordered step, 512
    // 1223 us, 1024 1233 us, 64 1276 us)
    __builtin_amdgcn_s_sleep(8);
  }
}

// Add `tiles` finished tiles of phase ph to every replica of its counter,
// one replica per lane of the calling wave (one instruction instead of
// kOrdReplicas from one lane: 1250 -> 1235 us per ordered step; no return
// value: nothing waits for these atomics).
__device__ inline void count_phase_tiles(uint32_t* odone, int ph, uint32_t tiles, int lane) {
  if (lane < kOrdReplicas)
    __hip_atomic_fetch_add(odone + ((size_t)ph * kOrdReplicas + lane) * kOrdLineWords, tiles, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// y[row0 .. row0+3] of one batch row = fp16(v * scale) (+ bias) for the rows
// below n (sc: the four rows' fp16 scales).  When all four rows exist and y
// is 8-byte aligned, one 8-byte store (and one 8-byte bias load) instead of
// four 2-byte ones.
__device__ __forceinline__ void store_rows4(uint16_t* yr, const uint16_t* bias, int row0, int n, const float v[4],
                                            u32x2_t sc) {
  uint16_t out[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) out[j] = f2h(v[j] * h2f((uint16_t)(sc[j >> 1] >> (16 * (j & 1)))));
  if (row0 + 4 <= n && ((reinterpret_cast<uintptr_t>(yr + row0) | reinterpret_cast<uintptr_t>(bias + row0)) & 7) == 0) {
    if (bias) {
      const u32x2_t bw = *(const TP_GLOBAL u32x2_t*)(bias + row0);
#pragma unroll
      for (int j = 0; j < 4; ++j) out[j] = f2h(h2f(out[j]) + h2f((uint16_t)(bw[j >> 1] >> (16 * (j & 1)))));
    }
    const u32x2_t w = {(uint32_t)out[0] | ((uint32_t)out[1] << 16), (uint32_t)out[2] | ((uint32_t)out[3] << 16)};
    *(TP_GLOBAL u32x2_t*)(yr + row0) = w;
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (row0 + j >= n) continue;
      uint16_t o = out[j];
      if (bias) o = f2h(h2f(o) + h2f(gld(bias + row0 + j)));
      gst(yr + row0 + j, o);
    }
  }
}

// Where one block of the ordered schedule sits, and the wave's chunk of it
// (scalar values, read one block ahead).
struct OrdDesc {
  bool valid;
  int li, t0, nt, G4, N, ph;
  int c0, nu;  // the wave's chunk: flat units [c0, c0 + nu) of the block
  int tc, k0;  // tile and K unit of flat unit c0
  __amdgpu_buffer_rsrc_t prs, mrs, srs;
  uint32_t zoff, zld;
  const uint16_t* bias;
  uint16_t* y;
  int n, ldy;
};

template <int MW>
__device__ __forceinline__ OrdDesc ord_desc(const StackRO& P, int blk, int total, int wave, const char* zbuf) {
  constexpr uint32_t unit_p = 4u * kTileRows * 8u;
  constexpr uint32_t unit_m = 4u * kTileRows * MW * 4u;
  OrdDesc D;
  D.valid = blk < total;
  const TP_CONST OrdBlockDesc& E = cread(P.oblk + (D.valid ? blk : 0));
  D.li = E.li;
  D.t0 = E.t0;
  D.nt = D.valid ? E.nt : 0;
  const TP_CONST LinearDesc& L = cread(P.lin + D.li);
  D.G4 = L.G4;
  D.N = D.nt * D.G4;
  D.c0 = (wave * D.N) >> 3;  // 8 waves
  D.nu = (((wave + 1) * D.N) >> 3) - D.c0;
  D.tc = D.c0 / D.G4;
  D.k0 = D.c0 - D.tc * D.G4;
  D.ph = cread(P.lphase + D.li);
  D.prs = buffer_rsrc(reinterpret_cast<const char*>(L.path) + (size_t)D.t0 * D.G4 * unit_p,
                      (uint32_t)D.N * unit_p);
  D.mrs = buffer_rsrc(reinterpret_cast<const char*>(L.member) + (size_t)D.t0 * D.G4 * unit_m,
                      (uint32_t)D.N * unit_m);
  D.srs = buffer_rsrc(L.scales, (uint32_t)L.n * 2u);
  D.zoff = (uint32_t)(reinterpret_cast<const char*>(L.z) - zbuf);
  D.zld = (uint32_t)D.G4 * kChunkCols;
  D.bias = L.bias;
  D.y = L.y;
  D.n = L.n;
  D.ldy = L.ldy;
  return D;
}

// Registers of one block: UMAX units in flight (a rolling window over the
// wave's chunk), the halo word (path word 1 of the unit before the chunk,
// K block 3 lanes) and the row scales of the tiles the wave finishes.
template <int MW, int NZ, int UMAX>
struct OrdRegs {
  UnitRegs<MW, NZ> R[UMAX];
  uint32_t x1_prev;
  u32x2_t sc[kOrdFinish];
};

// Loads of flat unit f (K unit k) of the block into R (past the wave's
// chunk: out of range, no memory traffic).  zv: the lane's z offsets inside
// a unit (out of range for batch rows past the batch).
template <int MW, int NZ>
__device__ __forceinline__ void ord_unit(UnitRegs<MW, NZ>& R, const OrdDesc& D, int f, int k, uint32_t pv,
                                         uint32_t mv, const uint32_t* zv, __amdgpu_buffer_rsrc_t zrs) {
  constexpr uint32_t unit_p = 4u * kTileRows * 8u;
  constexpr uint32_t unit_m = 4u * kTileRows * MW * 4u;
  constexpr uint32_t unit_z = kChunkCols * 2u;
  const bool ok = f < D.c0 + D.nu;
  const uint32_t fu = (uint32_t)(ok ? f : 0), ku = (uint32_t)(ok ? k : 0);
  R.X = __builtin_amdgcn_raw_buffer_load_b64(D.prs, ok ? pv : kOutOfRange, fu * unit_p, weight_policy(MW));
  R.M = MemberBuf<MW>::load(D.mrs, ok ? mv : kOutOfRange, fu * unit_m);
#pragma unroll
  for (int l = 0; l < NZ; ++l)
    R.Z[l] = __builtin_amdgcn_raw_buffer_load_b128(zrs, ok ? zv[l] : kOutOfRange, D.zoff + ku * unit_z, 0);
}

// K unit after k in a tile of G4 units (wrapping to the next tile).
__device__ __forceinline__ int ord_next_k(int k, int G4) { return k + 1 == G4 ? 0 : k + 1; }

// A block's first loads: halo word and scales (oldest, so that waiting for
// them waits for nothing else of the block), then the chunk's first UMAX
// units.
template <int MW, int NZ, int UMAX>
__device__ __forceinline__ void ord_head(OrdRegs<MW, NZ, UMAX>& B, const OrdDesc& D, int wave, uint32_t pv,
                                         uint32_t mv, const uint32_t* zv, int q, __amdgpu_buffer_rsrc_t zrs) {
  constexpr uint32_t unit_p = 4u * kTileRows * 8u;
  B.x1_prev = __builtin_amdgcn_raw_buffer_load_b32(D.prs, (D.nu > 0 && D.k0 > 0) ? pv + 4u : kOutOfRange,
                                                   (uint32_t)(D.k0 > 0 ? D.c0 - 1 : 0) * unit_p, 0);
#pragma unroll
  for (int i = 0; i < kOrdFinish; ++i) {
    const int t = wave + i * kWavesPerGroup;
    B.sc[i] = load_rows4(D.srs, (D.t0 + t) * kTileRows + 4 * q, D.n, t < D.nt);
  }
  int k = D.k0;
#pragma unroll
  for (int u = 0; u < UMAX; ++u) {
    ord_unit<MW, NZ>(B.R[u], D, D.c0 + u, k, pv, mv, zv, zrs);
    k = ord_next_k(k, D.G4);
  }
}

// The lane's z offsets inside a unit of a block (batch rows past the batch:
// out of range).
template <int NZ>
__device__ __forceinline__ void ord_zv(uint32_t* zv, const OrdDesc& D, int q, int slot, int bb, int batch) {
  constexpr int SLOTS = 4;
#pragma unroll
  for (int l = 0; l < NZ; ++l)
    zv[l] = bb < batch ? ((uint32_t)bb * D.zld + (uint32_t)(q * kSegCols + mfma_col(l * SLOTS + slot))) * 2u
                       : kOutOfRange;
}

// A wave's partial sum of one tile into LDS: accumulator `slot` holds this
// lane's column; the slots of each batch row are summed and the 16 (K
// block, batch row) sums land in the slot-0 lanes.
template <int SLOTS, int SB>
__device__ __forceinline__ void ord_flush(float4_t* acc, float4_t* dst, int slot, int pl) {
  const float4_t v = slot_column_sums<SLOTS, SB>(acc);  // (valid in the slot-0 lanes)
#pragma unroll
  for (int k = 0; k < SLOTS; ++k) acc[k] = float4_t{0.f, 0.f, 0.f, 0.f};
  if (slot == 0) dst[pl] = v;
}

template <int KB, int NS>
__global__ void __launch_bounds__(kGroupThreads) __attribute__((amdgpu_waves_per_eu(4)))
tcq_stack_ordered_kernel(const char* __restrict__ plan_ro, char* __restrict__ plan_rw,
                         const uint16_t* __restrict__ codebook, int spin_limit) {
  constexpr int SB = 4, SLOTS = 4, NZ = 2;
  constexpr int MW = member_words(KB);
  constexpr int UMAX = ord_max_units(KB);
  __shared__ __attribute__((aligned(16))) uint32_t table[kTableWords];
  // partial sums: [wave][tile % kOrdSegs][(K block, batch row)]
  __shared__ __attribute__((aligned(16))) float4_t part[kWavesPerGroup][kOrdSegs][16];
  const StackRO P = stack_ro(plan_ro);
  const TP_CONST StackInfo& info = cread(P.info);
  StackCounters* C = reinterpret_cast<StackCounters*>(plan_rw);
  uint32_t* odone = reinterpret_cast<uint32_t*>(plan_rw + P.odone);
  const int batch = info.batch;
  const int total = info.total_k;
  if (batch > SB || info.n_rot <= 0) {  // not a plan for this kernel: refuse uniformly
    if (threadIdx.x == 0 && blockIdx.x == 0) atomicExch(&C->error, 2u);
    return;
  }
  const char* zbuf = plan_rw + P.zbuf;
  const __amdgpu_buffer_rsrc_t zrs = buffer_rsrc(zbuf, (uint32_t)info.zbuf_bytes);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, q = lane >> 4;
  const int slot = r / SB, bb = r % SB;
  const int pl = q * 4 + bb;  // this lane's (K block, batch row) sum in the slot-0 lanes
  const uint32_t laneoff = lane_offsets<KB>(lane);
  const uint32_t pv = (uint32_t)(q * kTileRows + r) * 8u;
  const uint32_t mv = (uint32_t)(q * kTileRows + r) * MW * 4u;
  const uint32_t cb_lane = gld(codebook + (lane & ((2 << KB) - 1)));
  const int rep = (int)blockIdx.x % kOrdReplicas;
  uint32_t gen = 0;
  if (tid == 0) gen = __hip_atomic_load(&C->gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  int blk = blockIdx.x;
  OrdDesc D = ord_desc<MW>(P, blk, total, wave, zbuf);
  OrdRegs<MW, NZ, UMAX> B;
  uint32_t zv[NZ];
  ord_zv<NZ>(zv, D, q, slot, bb, batch);
  if (D.valid) ord_head<MW, NZ, UMAX>(B, D, wave, pv, mv, zv, q, zrs);
  OrdDesc Dn = ord_desc<MW>(P, blk + gridDim.x, total, wave, zbuf);
  build_pair_table_lanes<KB>(table, cb_lane, tid, kGroupThreads);
  uint32_t done_tiles = 0;  // wave 0: tiles of phase D.ph finished, not yet counted
  int open_ph = 0;          // phases up to this one are open to this workgroup

  while (D.valid) {
    if (D.ph > open_ph) {  // (a workgroup's blocks come in phase order)
      if (tid == 0) wait_phase_replica(P, odone, C, D.ph, gen, rep, spin_limit);
      open_ph = D.ph;
    }
    __syncthreads();  // (also: the last block's reads of `part` are done)
    float4_t acc[SLOTS];
#pragma unroll
    for (int k = 0; k < SLOTS; ++k) acc[k] = float4_t{0.f, 0.f, 0.f, 0.f};
    // The chunk through a rolling window of UMAX register sets: the first
    // UMAX units were loaded before the phase wait; in longer chunks the set
    // a unit frees is reloaded with the unit UMAX further on.  A tile that
    // ends inside the chunk leaves its partial sum in LDS.
    uint32_t prev = B.x1_prev;
    int kd = D.k0, td = D.tc;  // K unit and tile of the unit decoded next
    int kl = D.k0;             // K unit of the unit reloaded next
#pragma unroll
    for (int u = 0; u < UMAX; ++u) kl = ord_next_k(kl, D.G4);
    for (int base = 0; base < D.nu; base += UMAX) {
      const bool more = base + UMAX < D.nu;  // (wave-uniform)
#pragma unroll
      for (int u = 0; u < UMAX; ++u) {
        if (base + u < D.nu) {
          if (kd == 0) prev = 0u;  // a tile starts: no halo
          const uint32_t provide = (q == 3) ? prev : B.R[u].X[1];
          slot_unit<KB, NS, SB, MW, NZ>(B.R[u], provide, lane, laneoff, table, acc);
          prev = B.R[u].X[1];
          kd = ord_next_k(kd, D.G4);
          if (kd == 0) ord_flush<SLOTS, SB>(acc, part[wave][td++ % kOrdSegs], slot, pl);
        }
        if (more) {
          ord_unit<MW, NZ>(B.R[u], D, D.c0 + base + UMAX + u, kl, pv, mv, zv, zrs);
          kl = ord_next_k(kl, D.G4);
        }
      }
    }
    if (D.nu > 0 && kd != 0) ord_flush<SLOTS, SB>(acc, part[wave][td % kOrdSegs], slot, pl);
    // Every load of the block has been consumed or was out of range (those
    // return at once): an explicit wait tells the compiler so, and keeps its
    // own waits out of the y stores and the next block's loads below.
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    // Wave w finishes tiles w, w + 8, w + 16: the partial sums of the waves
    // whose chunks meet the tile, in wave order.
#pragma unroll
    for (int i = 0; i < kOrdFinish; ++i) {
      const int t = wave + i * kWavesPerGroup;
      if (t < D.nt && slot == 0) {
        float4_t v = float4_t{0.f, 0.f, 0.f, 0.f};
        const int ta = t * D.G4, tb = ta + D.G4;  // the tile's flat units
        for (int w = 0; w < kWavesPerGroup; ++w) {
          const int a = (w * D.N) >> 3, b = ((w + 1) * D.N) >> 3;
          if (a < b && a < tb && b > ta) {
            const float4_t s = part[w][t % kOrdSegs][pl];
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] += s[j];
          }
        }
        if (bb < batch) {
          const float vv[4] = {v[0], v[1], v[2], v[3]};
          store_rows4(D.y + (size_t)bb * D.ldy, D.bias, (D.t0 + t) * kTileRows + 4 * q, D.n, vv, B.sc[i]);
        }
      }
    }
    // The next block's loads go out at once when it belongs to this phase or
    // one of the next two (one: 1222 us per step, two: 1217, three: 1221).
    // For a later phase they wait until the phase before it is open: all
    // workgroups end a phase together, and loads for far-off phases issued
    // then would queue ahead of the stores and loads of the phases that run
    // first.
    // The last block of the phase in this workgroup counts its tiles as soon
    // as the y stores of every wave are complete, and only then issues the
    // next block's loads: issued first, they met a full memory pipeline at
    // the phase end and held the count back (1297 -> 1245 us per step).
    const bool near = Dn.valid && Dn.ph <= D.ph + 2;
    const bool last = !Dn.valid || Dn.ph != D.ph;
    if (near && !last) {
      ord_zv<NZ>(zv, Dn, q, slot, bb, batch);
      ord_head<MW, NZ, UMAX>(B, Dn, wave, pv, mv, zv, q, zrs);
    }
    if (wave == 0) done_tiles += (uint32_t)D.nt;
    if (last) {
      __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (wave == 0) {
        count_phase_tiles(odone, D.ph, done_tiles, lane);
        done_tiles = 0;
      }
      if (near) {
        ord_zv<NZ>(zv, Dn, q, slot, bb, batch);
        ord_head<MW, NZ, UMAX>(B, Dn, wave, pv, mv, zv, q, zrs);
      }
    }
    if (Dn.valid && !near) {
      if (tid == 0) wait_phase_replica(P, odone, C, Dn.ph - 1, gen, rep, spin_limit);
      __syncthreads();
      ord_zv<NZ>(zv, Dn, q, slot, bb, batch);
      ord_head<MW, NZ, UMAX>(B, Dn, wave, pv, mv, zv, q, zrs);
    }
    D = Dn;
    blk += gridDim.x;
    Dn = ord_desc<MW>(P, blk + gridDim.x, total, wave, zbuf);
  }

  // The last workgroup out resets the launch counters and opens the next
  // launch's generation.
  if (tid == 0) {
    const uint32_t ex = atomicAdd(&C->exited, 1u);
    if (ex == gridDim.x - 1) {
      atomicExch(&C->ticket, 0u);
      atomicExch(&C->exited, 0u);
      atomicAdd(&C->gen, 1u);
    }
  }
}

// ---------------------------------------------------------------------------
// 3. wide kernel (stack: batch 5..32; one linear: batch 9..32)
// ---------------------------------------------------------------------------
// One workgroup of 16 waves per CU takes *wide blocks* (16 row tiles x the
// full K of one linear) by ticket; wave w owns tile w.  The linear's rotated
// activations (the plan's z buffer, written by the rotation launch) pass
// through LDS in chunks of 512 columns x up to 32 batch rows, double
// buffered: while a chunk is decoded and multiplied, the next one is loaded
// into registers, then stored to the other buffer before the chunk's one
// barrier.  Per unit a wave decodes 4096 weights once and issues 8 MFMAs per
// 16-column batch tile against B operands read from LDS.
constexpr int kWideWaves = 16;
constexpr int kWideThreads = 64 * kWideWaves;
constexpr int kWideChunkHalves = 32 * kZCols;  // one staged chunk (32 rows x 512 columns)

// Path/member words of one chunk (kMaxUnitsPerBlock units) of one lane.
template <int MW>
struct ChunkRegs {
  uint2 X[kMaxUnitsPerBlock];
  uint32_t M[kMaxUnitsPerBlock][MW];
};

template <int MW>
__device__ __forceinline__ ChunkRegs<MW> load_chunk(const LinearDesc& L, const uint32_t* pt, const uint32_t* mt,
                                                     int ch, int q, int r) {
  // Branch-free: units past the block's K range (and inactive waves, whose
  // pointers address tile 0) reload unit 0 of the chunk; they are never used.
  ChunkRegs<MW> c;
  const int gu0 = ch * kMaxUnitsPerBlock;
  const int ngu = min(kMaxUnitsPerBlock, L.G4 - gu0);
#pragma unroll
  for (int u = 0; u < kMaxUnitsPerBlock; ++u) {
    const int g = 4 * (gu0 + (u < ngu ? u : 0)) + q;
    c.X[u] = gld2_w<MW>(pt + (g * kTileRows + r) * 2);
#pragma unroll
    for (int i = 0; i < MW; ++i) c.M[u][i] = gld_w<MW>(mt + (g * kTileRows + r) * MW + i);
  }
  return c;
}

// A staged chunk is 2048 16-byte pieces: NP = 2048 / NT per thread of an
// NT-thread workgroup.
template <int NP>
struct ZChunkN {
  u32x4_t v[NP];
};
typedef ZChunkN<2> ZChunk;

// Thread tid's pieces of chunk ch: piece i = tid + NT k is row i / 64,
// columns 8 (i % 64) ..; rows past the batch are not loaded.
template <int NT = kWideThreads>
__device__ __forceinline__ ZChunkN<2048 / NT> wide_load_z(__amdgpu_buffer_rsrc_t zrs, int zld, int batch, int ch,
                                                          int tid) {
  ZChunkN<2048 / NT> c;
#pragma unroll
  for (int k = 0; k < 2048 / NT; ++k) {
    const int i = tid + NT * k;
    const int row = i >> 6, c8 = (i & 63) * 8;
    const uint32_t off = row < batch ? (uint32_t)(row * zld + ch * kZCols + c8) * 2u : kOutOfRange;
    c.v[k] = __builtin_amdgcn_raw_buffer_load_b128(zrs, off, 0, 0);
  }
  return c;
}

// (lcol: the lane's group of 8 columns -- the lane itself, or its
// wide_rotate relabeling)
template <int NT = kWideThreads>
__device__ __forceinline__ void wide_store_z(uint16_t* zb, const ZChunkN<2048 / NT>& c, int batch, int tid,
                                             int lcol) {
#pragma unroll
  for (int k = 0; k < 2048 / NT; ++k) {
    const int i = tid + NT * k;
    const int row = i >> 6, c8 = lcol * 8;
    if (row < batch) *reinterpret_cast<u32x4_t*>(zb + zl_index(row, c8)) = c.v[k];
  }
}

// ROT (per-linear launches at Hadamard blocks <= 512, every chunk then a
// whole number of blocks): thread tid's two 8-column pieces (columns
// 8 lcol ..) of chunk ch of the unrotated input and of rot_scale (columns
// past d read as zero).
struct XChunk {
  u32x4_t x[2], r[2];
};
__device__ __forceinline__ XChunk wide_load_x(const LinearDesc& L, int batch, int ch, int tid, int lcol) {
  const __amdgpu_buffer_rsrc_t xrs = buffer_rsrc(L.x, (uint32_t)(batch * L.ldx) * 2u);
  const __amdgpu_buffer_rsrc_t rrs = buffer_rsrc(L.rs, (uint32_t)L.d * 2u);
  XChunk c;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int i = tid + kWideThreads * k;
    const int row = i >> 6, col = ch * kZCols + lcol * 8;
    const bool in = row < batch && col < L.d;  // d % 8 == 0: a piece is wholly in or out
    c.x[k] = __builtin_amdgcn_raw_buffer_load_b128(xrs, in ? (uint32_t)(row * L.ldx + col) * 2u : kOutOfRange, 0, 0);
    c.r[k] = __builtin_amdgcn_raw_buffer_load_b128(rrs, in ? (uint32_t)col * 2u : kOutOfRange, 0, 0);
  }
  return c;
}

// The lane's group of 8 columns in wide_rotate's pieces: the relabeling of
// the tile transform (rot_lane_index), so that every lane stage below
// distance 128 is one DPP move.
__device__ __forceinline__ int wide_lane_col(int lane) { return rot_lane_index(lane); }

// z = fp16(blockFWHT(x * rot_scale) / sqrt(hb)) of the pieces: a wave holds
// one row's 512 columns (8 per lane, columns 8 wide_lane_col ..), so the
// butterflies at distance 1..4 run in registers and 8..256 across lanes, in
// increasing distance as the reference's transform, all in fp32, one
// rounding to fp16 -- the steps of the tile transform (tp_rotate_tile.h):
// the products fused into the distance-1 stage as v_fma_mix_f32, each lane
// stage one DPP move (bpermute at distance 128, 256: a permlane swap there,
// which writes both of its registers, pushed this kernel into scratch) and
// one FMA.  (One
// path for every block size, stages tested at run time: a second,
// unrolled path for 512-column blocks pushed the kernel into scratch.)
template <int K>
__device__ __forceinline__ void wide_lane_stage(float* v, int m, int lane4, int hb) {
  if ((8 << K) < hb) {
    const float sg = __builtin_bit_cast(float, 0x3F800000u | (((uint32_t)m << (31 - K)) & 0x80000000u));
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = __builtin_fmaf(sg, v[e], rot_partner<K>(v[e], lane4));
  }
}
__device__ __forceinline__ ZChunk wide_rotate(const XChunk& c, int lane, int hb, float hdiv) {
  ZChunk z;
  const float rdiv = 1.f / hdiv;
  const int m = rot_lane_index(lane), lane4 = 4 * lane;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const u32x2_t xw[2] = {u32x2_t{c.x[k][0], c.x[k][1]}, u32x2_t{c.x[k][2], c.x[k][3]}};
    const u32x2_t rw[2] = {u32x2_t{c.r[k][0], c.r[k][1]}, u32x2_t{c.r[k][2], c.r[k][3]}};
    float v[8];
    if (hb > 1) rot_products<true, 2>(xw, rw, v);  // with distance 1
    else rot_products<false, 2>(xw, rw, v);
#pragma unroll
    for (int h = 2; h < 8; h <<= 1) {  // distances 2, 4
      if (h < hb) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if ((e & h) == 0) {
            const float a = v[e], b = v[e + h];
            v[e] = a + b;
            v[e + h] = a - b;
          }
        }
      }
    }
    wide_lane_stage<0>(v, m, lane4, hb);  // distance 8
    wide_lane_stage<1>(v, m, lane4, hb);
    wide_lane_stage<2>(v, m, lane4, hb);
    wide_lane_stage<3>(v, m, lane4, hb);
    wide_lane_stage<4>(v, m, lane4, hb);
    wide_lane_stage<5>(v, m, lane4, hb);  // distance 256
    // (the corrected reciprocal is exact for a power-of-two root as well)
#pragma unroll
    for (int e = 0; e < 4; ++e)
      z.v[k][e] = pack_h2(div_by_block_root(v[2 * e], hdiv, rdiv), div_by_block_root(v[2 * e + 1], hdiv, rdiv));
  }
  return z;
}

// One unit of one wave of the wide kernel: decode 64 weights per lane, then
// for each of the 8 MFMA positions read the B operands of the NBT batch tiles
// from the staged chunk (rows past the batch hold stale data: their MFMA
// columns are never written out).  PREB: position p + 1's B reads are issued
// before position p's MFMAs, so that not every position waits for an LDS
// round trip (the scheduler would otherwise place each read next to its
// MFMA to save the registers; batch-32 stack GEMV 524 -> 513 us).  The
// rotating per-linear variants whose registers are full (4-bit, and 32 rows
// with 4 trellis states) keep the plain order.
template <int KB, int NS, int NBT, bool PREB = true>
__device__ __forceinline__ void wide_unit(const uint2 X, const uint32_t* Mw, const uint32_t x1_last, const int gu,
                                          const int lc, const int q, const int r, const int lane,
                                          const uint32_t laneoff, const uint32_t* table, const uint16_t* zb,
                                          float4_t* acc) {
  const uint32_t provide = (q == 3) ? (gu == 0 ? 0u : x1_last) : X.y;
  const uint32_t halo = (uint32_t)__shfl((int)provide, (lane + 48) & 63, 64);
  const uint32_t P = ((halo >> 1) & 0x55555555u) | ((X.y << 1) & 0xAAAAAAAAu);
  MemberWords<KB> m[2];
  split_members<KB>(Mw, m);
  // column offset (halves) of MFMA position pos = 4 x + j in the segment
  auto boff = [](int pos) { return 16 * (pos >> 2) + (pos & 2 ? 32 : 0) + (pos & 1 ? 8 : 0); };
  half8_t bcur[NBT];
  if constexpr (PREB) {
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt)
      bcur[bt] = *reinterpret_cast<const half8_t*>(zb + zl_index(bt * 16 + r, lc + boff(0)));
  }
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    u32x4_t A[4];
    decode_word<KB, NS>(x ? X.y : X.x, x ? X.x : P, m[x], table, laneoff, A);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int pos = 4 * x + j;
      const half8_t av = __builtin_bit_cast(half8_t, A[j]);
      if constexpr (PREB) {
        half8_t bnext[NBT];
        if (pos < 7) {
#pragma unroll
          for (int bt = 0; bt < NBT; ++bt)
            bnext[bt] = *reinterpret_cast<const half8_t*>(zb + zl_index(bt * 16 + r, lc + boff(pos + 1)));
        }
        __builtin_amdgcn_sched_barrier(0);  // (the reads stay ahead of the MFMAs)
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) acc[bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bcur[bt], acc[bt], 0, 0, 0);
        if (pos < 7) {
#pragma unroll
          for (int bt = 0; bt < NBT; ++bt) bcur[bt] = bnext[bt];
        }
      } else {
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) {
          const half8_t b = *reinterpret_cast<const half8_t*>(zb + zl_index(bt * 16 + r, lc + boff(pos)));
          acc[bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b, acc[bt], 0, 0, 0);
        }
      }
    }
  }
}

// The same unit for two row tiles of one wave (the unit at the same K of
// both): each B operand read from the staged chunk feeds the MFMAs of both
// tiles, half the LDS reads of two waves with one tile each.
template <int KB, int NS, int NBT>
__device__ __forceinline__ void wide_unit2(const uint2 X0, const uint32_t* M0, const uint32_t x1l0, const uint2 X1,
                                           const uint32_t* M1, const uint32_t x1l1, const int gu, const int lc,
                                           const int q, const int r, const int lane, const uint32_t laneoff,
                                           const uint32_t* table, const uint16_t* zb, float4_t (*acc)[NBT]) {
  const uint32_t h0 = (uint32_t)__shfl((int)((q == 3) ? (gu == 0 ? 0u : x1l0) : X0.y), (lane + 48) & 63, 64);
  const uint32_t h1 = (uint32_t)__shfl((int)((q == 3) ? (gu == 0 ? 0u : x1l1) : X1.y), (lane + 48) & 63, 64);
  const uint32_t P0 = ((h0 >> 1) & 0x55555555u) | ((X0.y << 1) & 0xAAAAAAAAu);
  const uint32_t P1 = ((h1 >> 1) & 0x55555555u) | ((X1.y << 1) & 0xAAAAAAAAu);
  MemberWords<KB> m0[2], m1[2];
  split_members<KB>(M0, m0);
  split_members<KB>(M1, m1);
  auto boff = [](int pos) { return 16 * (pos >> 2) + (pos & 2 ? 32 : 0) + (pos & 1 ? 8 : 0); };
  half8_t bcur[NBT];
#pragma unroll
  for (int bt = 0; bt < NBT; ++bt)
    bcur[bt] = *reinterpret_cast<const half8_t*>(zb + zl_index(bt * 16 + r, lc + boff(0)));
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    u32x4_t A0[4], A1[4];
    decode_word<KB, NS>(x ? X0.y : X0.x, x ? X0.x : P0, m0[x], table, laneoff, A0);
    decode_word<KB, NS>(x ? X1.y : X1.x, x ? X1.x : P1, m1[x], table, laneoff, A1);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int pos = 4 * x + j;
      half8_t bnext[NBT];
      if (pos < 7) {
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt)
          bnext[bt] = *reinterpret_cast<const half8_t*>(zb + zl_index(bt * 16 + r, lc + boff(pos + 1)));
      }
      __builtin_amdgcn_sched_barrier(0);  // (the reads stay ahead of the MFMAs)
#pragma unroll
      for (int bt = 0; bt < NBT; ++bt) {
        acc[0][bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, A0[j]), bcur[bt],
                                                            acc[0][bt], 0, 0, 0);
        acc[1][bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, A1[j]), bcur[bt],
                                                            acc[1][bt], 0, 0, 0);
      }
      if (pos < 7) {
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) bcur[bt] = bnext[bt];
      }
    }
  }
}

// Wide block wb of linear L over 512-column chunks [ch0, ch1): z rows at
// z + b * zld (fp16, zero past d).  The full K range writes y; a part of it
// adds its sums into the linear's workspace with device-scope atomics, and
// the wave that completes a tile's K range (counted per tile) writes y and
// clears the sums (the split-K protocol of tcq_gemv_tiled_kernel).
// build_table: the pair table is built here (from cb_lane), after the first
// chunk's z and weight loads are issued, so that neither waits for it.
// ROT: z is computed from L.x and L.rs chunk by chunk (wide_rotate).
template <int KB, int NS, int NBT, bool ROT = false, int TPW = 1>
__device__ void wide_block(const LinearDesc& L, int wb, int ch0, int ch1, const uint16_t* z, int zld, int batch,
                           uint16_t* zl, uint32_t* table, uint32_t laneoff, int tid, int wave, int lane,
                           bool build_table = false, uint32_t cb_lane = 0) {
  // TPW tiles per wave (a workgroup of kWideWaves / TPW waves covers the
  // block's 16 tiles): tile k of a wave is wb * 16 + wave + k * 16 / TPW.
  static_assert(TPW == 1 || (TPW == 2 && !ROT), "two tiles per wave: stack (z staged) only");
  constexpr int NT = kWideThreads / TPW;
  constexpr int NWV = kWideWaves / TPW;
  constexpr int MW = member_words(KB);
  const int r = lane & 15, q = lane >> 4;
  const int nch = (L.G4 + kMaxUnitsPerBlock - 1) / kMaxUnitsPerBlock;
  int t[TPW];
  bool active[TPW];
  const uint32_t* pt[TPW];
  const uint32_t* mt[TPW];
#pragma unroll
  for (int k = 0; k < TPW; ++k) {
    t[k] = wb * kWideWaves + wave + NWV * k;
    active[k] = t[k] < L.T;
    pt[k] = L.path + (size_t)(active[k] ? t[k] : 0) * L.G * (kTileRows * 2);
    mt[k] = L.member + (size_t)(active[k] ? t[k] : 0) * L.G * (kTileRows * MW);
  }
  const __amdgpu_buffer_rsrc_t zrs = buffer_rsrc(z, (uint32_t)(batch * zld) * 2u);

  float4_t acc[TPW][NBT];
#pragma unroll
  for (int k = 0; k < TPW; ++k)
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt) acc[k][bt] = float4_t{0.f, 0.f, 0.f, 0.f};
  // halo of the range's first unit: word 1 of the previous unit's last segment
  uint32_t x1_last[TPW];
#pragma unroll
  for (int k = 0; k < TPW; ++k)
    x1_last[k] = ch0 > 0 ? pt[k][((4 * ch0 * kMaxUnitsPerBlock - 1) * kTileRows + r) * 2 + 1] : 0u;
  // the epilogue's row scales and bias (rows 4q..4q+3 of the tile, zeros
  // past n), loaded now so that they are in registers when the sums are --
  // except in the 4-bit, 32-row, rotating variant, whose registers are full:
  // there they would be spilled to scratch and reloaded (a round trip of
  // its own), so they load in the epilogue
  constexpr bool kEarlyEpilogue = !(KB == 4 && NBT == 2 && ROT);
  int row0[TPW];
  u32x2_t sc4[TPW], bs4[TPW];
  const __amdgpu_buffer_rsrc_t srs = buffer_rsrc(L.scales, (uint32_t)L.n * 2u);
  const __amdgpu_buffer_rsrc_t brs = buffer_rsrc(L.bias, L.bias ? (uint32_t)L.n * 2u : 0u);
#pragma unroll
  for (int k = 0; k < TPW; ++k) {
    row0[k] = t[k] * kTileRows + 4 * q;
    sc4[k] = u32x2_t{0u, 0u};
    bs4[k] = u32x2_t{0u, 0u};
    if constexpr (kEarlyEpilogue) {
      sc4[k] = load_rows4(srs, row0[k], L.n, active[k]);
      bs4[k] = load_rows4(brs, row0[k], L.n, active[k] && L.bias);
    }
  }
  // The first chunk's z, then its weights: the z staging waits for the z
  // loads only, and the weights are in flight during it (and during the
  // table build).
  ZChunkN<2048 / NT> c0;
  XChunk x0;
  const int lcol = ROT ? wide_lane_col(lane) : lane;  // the lane's z columns in a chunk
  if constexpr (ROT) x0 = wide_load_x(L, batch, ch0, tid, lcol);
  else c0 = wide_load_z<NT>(zrs, zld, batch, ch0, tid);
  ChunkRegs<MW> ra[TPW];
#pragma unroll
  for (int k = 0; k < TPW; ++k) ra[k] = load_chunk<MW>(L, pt[k], mt[k], ch0, q, r);
  if (build_table) build_pair_table_lanes<KB>(table, cb_lane, tid, NT);
  if constexpr (ROT) c0 = wide_rotate(x0, lane, L.hb, L.hdiv);
  wide_store_z<NT>(zl + (ch0 & 1) * kWideChunkHalves, c0, batch, tid, lcol);
  __syncthreads();
  // Chunk ch: prefetch chunk ch + 1 of z, decode + multiply ch, store the
  // prefetch into the other buffer, one barrier (the next chunk's buffer is
  // full and nobody still reads the one it will overwrite).
  auto body = [&](int ch, const ChunkRegs<MW>* regs) {
    const bool more = ch + 1 < ch1;
    ZChunkN<2048 / NT> nx;
    XChunk nxx;
    if (more) {
      if constexpr (ROT) nxx = wide_load_x(L, batch, ch + 1, tid, lcol);
      else nx = wide_load_z<NT>(zrs, zld, batch, ch + 1, tid);
    }
    const uint16_t* zb = zl + (ch & 1) * kWideChunkHalves;
    // (with two tiles, the second is decoded whenever the first is active;
    // an inactive one reads tile 0's words and is never written out)
    if (active[0]) {
      const int gu0 = ch * kMaxUnitsPerBlock;
      const int ngu = min(kMaxUnitsPerBlock, L.G4 - gu0);
#pragma unroll
      for (int u = 0; u < kMaxUnitsPerBlock; ++u) {
        if (u < ngu) {
          const int gu = gu0 + u;
          const int lc = (4 * gu + q - 4 * gu0) * kSegCols;
          if constexpr (TPW == 1) {
            wide_unit<KB, NS, NBT, !(ROT && (KB == 4 || (NBT == 2 && NS == 4)))>(
                regs[0].X[u], regs[0].M[u], x1_last[0], gu, lc, q, r, lane, laneoff, table, zb, acc[0]);
          } else {
            wide_unit2<KB, NS, NBT>(regs[0].X[u], regs[0].M[u], x1_last[0], regs[1].X[u], regs[1].M[u],
                                    x1_last[1], gu, lc, q, r, lane, laneoff, table, zb, acc);
          }
#pragma unroll
          for (int k = 0; k < TPW; ++k) x1_last[k] = regs[k].X[u].y;
        }
      }
    }
    if (more) {
      if constexpr (ROT) nx = wide_rotate(nxx, lane, L.hb, L.hdiv);
      wide_store_z<NT>(zl + ((ch + 1) & 1) * kWideChunkHalves, nx, batch, tid, lcol);
    }
    __syncthreads();
  };
  for (int ch = ch0; ch < ch1; ch += 2) {
    ChunkRegs<MW> rb[TPW];
#pragma unroll
    for (int k = 0; k < TPW; ++k) rb[k] = load_chunk<MW>(L, pt[k], mt[k], ch + 1 < ch1 ? ch + 1 : ch, q, r);
    body(ch, ra);
    if (ch + 1 >= ch1) break;
#pragma unroll
    for (int k = 0; k < TPW; ++k) ra[k] = load_chunk<MW>(L, pt[k], mt[k], ch + 2 < ch1 ? ch + 2 : ch, q, r);
    body(ch + 1, rb);
  }

  // Epilogue: lane holds rows 4q..4q+3 of each of its tiles for batch column r.
#pragma unroll
  for (int k = 0; k < TPW; ++k) {
    if (!active[k]) continue;
    if constexpr (!kEarlyEpilogue) {
      sc4[k] = load_rows4(srs, row0[k], L.n, true);
      bs4[k] = load_rows4(brs, row0[k], L.n, L.bias != nullptr);
    }
    float v[NBT][4];
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
      for (int i = 0; i < 4; ++i) v[bt][i] = acc[k][bt][i];
    if (ch0 > 0 || ch1 < nch) {
      const int ldws = 16 * NBT;
#pragma unroll
      for (int bt = 0; bt < NBT; ++bt) {
        if (bt * 16 + r >= batch) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) atomicAdd(L.ws + (size_t)(row0[k] + i) * ldws + bt * 16 + r, v[bt][i]);
      }
      __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
      const uint32_t units = (uint32_t)(min(ch1 * kMaxUnitsPerBlock, L.G4) - ch0 * kMaxUnitsPerBlock);
      uint32_t old = 0;
      if (lane == 0) old = atomicAdd(L.cnt + t[k], units);
      old = (uint32_t)__shfl((int)old, 0, 64);
      if (old + units != (uint32_t)L.G4) continue;
      // Last contributor: read and clear the sums (also read-modify-write atomics).
#pragma unroll
      for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          v[bt][i] = (bt * 16 + r < batch) ? atomicExch(L.ws + (size_t)(row0[k] + i) * ldws + bt * 16 + r, 0.f)
                                           : 0.f;
      if (lane == 0) atomicExch(L.cnt + t[k], 0u);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = row0[k] + i;
      if (row >= L.n) continue;
      const float sc = h2f((uint16_t)(sc4[k][i >> 1] >> (16 * (i & 1))));
      const float bs = h2f((uint16_t)(bs4[k][i >> 1] >> (16 * (i & 1))));
#pragma unroll
      for (int bt = 0; bt < NBT; ++bt) {
        const int nb = bt * 16 + r;
        if (nb >= batch) continue;
        uint16_t out = f2h(v[bt][i] * sc);
        if (L.bias) out = f2h(h2f(out) + bs);
        gst(L.y + (size_t)nb * L.ldy + row, out);
      }
    }
  }
}

template <int KB, int NS, int NBT, int TPW = 1>
__global__ void __launch_bounds__(kWideThreads / TPW)
tcq_stack_wide_kernel(const char* __restrict__ plan_ro, char* __restrict__ plan_rw,
                      const uint16_t* __restrict__ codebook, int ordered, int spin_limit) {
  __shared__ __attribute__((aligned(16))) uint32_t table[kTableWords];
  extern __shared__ __attribute__((aligned(16))) uint16_t zl[];
  __shared__ int s_next;
  // Sizes come from the plan itself, never from the caller.
  const StackRO P = stack_ro(plan_ro);
  const int batch = P.info->batch;
  const int total = P.info->total_wide;
  StackCounters* C = reinterpret_cast<StackCounters*>(plan_rw);
  uint32_t* pdone = reinterpret_cast<uint32_t*>(plan_rw + P.pdone);
  if (batch > 16 * NBT || P.info->zbuf_bytes == 0) {  // not a plan for this kernel: refuse uniformly
    if (threadIdx.x == 0 && blockIdx.x == 0) atomicExch(&C->error, 2u);
    return;
  }
  const int32_t* sched = ordered ? P.sched_wo : P.sched_wu;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t laneoff = lane_offsets<KB>(lane);
  const uint32_t cb_lane = gld(codebook + (lane & ((2 << KB) - 1)));

  if (tid == 0) s_next = (int)atomicAdd(&C->ticket, 1u);
  build_pair_table_lanes<KB>(table, cb_lane, tid, kWideThreads / TPW);
  __syncthreads();
  int blk = __builtin_amdgcn_readfirstlane(s_next);

  while (blk < total) {
    const int e = sched[blk];
    const int li = __builtin_amdgcn_readfirstlane(e >> kStackBlockBits);
    const int wb = e & ((1 << kStackBlockBits) - 1);
    const LinearDesc L = P.lin[li];  // copied to registers once per block
    uint32_t next_ticket = 0;
    if (tid == 0) next_ticket = atomicAdd(&C->ticket, 1u);
    if (ordered) {
      const int ph = P.lphase[li];
      if (ph > 0) {
        if (tid == 0) wait_phase(P, pdone, C, ph, spin_limit);
        __syncthreads();
      }
    }
    wide_block<KB, NS, NBT, false, TPW>(L, wb, 0, (L.G4 + kMaxUnitsPerBlock - 1) / kMaxUnitsPerBlock, L.z,
                                        L.G4 * kChunkCols, batch, zl, table, laneoff, tid, wave, lane);
    if (ordered) {
      __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      // phase counts are in 8-tile blocks: a wide block covers two (one at the end)
      if (tid == 0) atomicAdd(&pdone[P.lphase[li]], (uint32_t)min(2, L.blocks - 2 * wb));
    }
    if (tid == 0) s_next = (int)next_ticket;
    __syncthreads();
    blk = __builtin_amdgcn_readfirstlane(s_next);
  }

  if (tid == 0) {
    const uint32_t ex = atomicAdd(&C->exited, 1u);
    if (ex == gridDim.x - 1) {
      for (int p = 0; p < P.info->n_phases; ++p) atomicExch(&pdone[p], 0u);
      atomicExch(&C->ticket, 0u);
      atomicExch(&C->exited, 0u);
    }
  }
}

// One linear at batch 9..32 with its rotated activations already in z
// (fp16 [batch][zld], zero past d): one workgroup per wide block.
template <int KB, int NS, int NBT, bool ROT>
__global__ void __launch_bounds__(kWideThreads)
tcq_wide_linear_kernel(const LinearDesc L, const uint16_t* __restrict__ z, int zld, int batch,
                       const uint16_t* __restrict__ codebook, int cps) {
  __shared__ __attribute__((aligned(16))) uint32_t table[kTableWords];
  extern __shared__ __attribute__((aligned(16))) uint16_t zl[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t laneoff = lane_offsets<KB>(lane);
  const uint32_t cb_lane = gld(codebook + (lane & ((2 << KB) - 1)));
  // workgroup (x, y) = (wide block, K part of cps chunks); the table is
  // built inside, once the first loads are in flight
  const int nch = (L.G4 + kMaxUnitsPerBlock - 1) / kMaxUnitsPerBlock;
  const int ch0 = (int)blockIdx.y * cps;
  wide_block<KB, NS, NBT, ROT>(L, (int)blockIdx.x, ch0, min(nch, ch0 + cps), z, zld, batch, zl, table, laneoff,
                               tid, wave, lane, true, cb_lane);
}

template <int KB, int NS>
void launch_wide_linear(const LinearDesc& L, const uint16_t* z, int zld, int batch, const uint16_t* cb,
                        hipStream_t s) {
  // Split K until the workgroups cover the CUs (down to one chunk per part;
  // fewer, longer parts measured slower despite fewer split-K atomics).
  const int groups = (L.T + kWideWaves - 1) / kWideWaves;
  const int nch = (L.G4 + kMaxUnitsPerBlock - 1) / kMaxUnitsPerBlock;
  const int want = (device_cu_count() + groups - 1) / groups;
  const int parts = L.ws ? std::max(1, std::min(nch, want)) : 1;
  const int cps = (nch + parts - 1) / parts;
  const dim3 grid(groups, (nch + cps - 1) / cps);
  const size_t zbytes = (size_t)2 * kWideChunkHalves * 2;
  auto kern = z ? (batch <= 16 ? tcq_wide_linear_kernel<KB, NS, 1, false> : tcq_wide_linear_kernel<KB, NS, 2, false>)
               : (batch <= 16 ? tcq_wide_linear_kernel<KB, NS, 1, true> : tcq_wide_linear_kernel<KB, NS, 2, true>);
  allow_dynamic_lds(reinterpret_cast<const void*>(kern), kTableBytes + 256);
  hipLaunchKernelGGL(kern, grid, dim3(kWideThreads), zbytes, s, L, z, zld, batch, cb, cps);
}

int linear_forward_wide(const LinearDesc& Lin, const uint16_t* z, int64_t zld, int64_t batch,
                        const uint16_t* codebook, int bits, int n_states, void* workspace, int64_t workspace_bytes,
                        hipStream_t s) {
  if (batch <= 8 || batch > 32) return kLinearNotHandled;
  // z null: rotate L.x * L.rs chunk by chunk in the launch (each 512-column
  // chunk a whole number of Hadamard blocks; 16-byte input pieces)
  if (!z && (Lin.hb > kZCols || Lin.d % 8 || Lin.ldx % 8 || ((uintptr_t)Lin.x & 15) || ((uintptr_t)Lin.rs & 15)))
    return kLinearNotHandled;
  // split-K sums: fp32 [T * 16 rows][16 * NBT] then one counter per tile
  LinearDesc L = Lin;
  const int64_t nbt = batch <= 16 ? 1 : 2;
  const int64_t sums = (int64_t)L.T * kTileRows * 16 * nbt * 4;
  if (workspace && workspace_bytes >= sums + (int64_t)L.T * 4 && !((uintptr_t)workspace & 15)) {
    L.ws = reinterpret_cast<float*>(workspace);
    L.cnt = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(workspace) + sums);
  } else {
    L.ws = nullptr;
    L.cnt = nullptr;
  }
  switch (bits * 100 + n_states) {
    case 204: launch_wide_linear<2, 4>(L, z, (int)zld, (int)batch, codebook, s); break;
    case 208: launch_wide_linear<2, 8>(L, z, (int)zld, (int)batch, codebook, s); break;
    case 216: launch_wide_linear<2, 16>(L, z, (int)zld, (int)batch, codebook, s); break;
    case 264: launch_wide_linear<2, 64>(L, z, (int)zld, (int)batch, codebook, s); break;
    case 304: launch_wide_linear<3, 4>(L, z, (int)zld, (int)batch, codebook, s); break;
    case 308: launch_wide_linear<3, 8>(L, z, (int)zld, (int)batch, codebook, s); break;
    case 316: launch_wide_linear<3, 16>(L, z, (int)zld, (int)batch, codebook, s); break;
    case 364: launch_wide_linear<3, 64>(L, z, (int)zld, (int)batch, codebook, s); break;
    case 404: launch_wide_linear<4, 4>(L, z, (int)zld, (int)batch, codebook, s); break;
    case 408: launch_wide_linear<4, 8>(L, z, (int)zld, (int)batch, codebook, s); break;
    case 416: launch_wide_linear<4, 16>(L, z, (int)zld, (int)batch, codebook, s); break;
    case 464: launch_wide_linear<4, 64>(L, z, (int)zld, (int)batch, codebook, s); break;
    default: return TP_ERR_UNSUPPORTED_STATES;
  }
  return launch_status();
}


// Each plan initialised in this process with a slot-kernel batch: its
// rotation tile count, blocks, batch and layout offsets.  A plan the process
// did not initialise gets kernels that read these from the plan header.
struct PlanReg {
  int n_rot_packed, n_rot_big;  // rotation tiles of blocks <= 4096 / above 4096
  int total, batch, total_k;
  int64_t lin_off, sched_o_off, sched_u_off;
};
std::mutex g_plan_mutex;
std::unordered_map<const void*, PlanReg> g_plans;

inline bool plan_lookup(const void* plan, PlanReg* out) {
  std::lock_guard<std::mutex> lock(g_plan_mutex);
  const auto it = g_plans.find(plan);
  if (it == g_plans.end()) return false;
  *out = it->second;
  return true;
}

template <int KB, int NS>
int launch_gemv(char* plan, int64_t total_blocks, int64_t batch, const uint16_t* cb, int ordered,
                int spin_limit, hipStream_t s) {
  const char* ro = plan + kStackRO;
  const int cus = device_cu_count();
  PlanReg reg;
  const bool known = plan_lookup(plan, &reg) && reg.batch == batch && reg.total == total_blocks;
  if (ordered && batch <= kSlotMaxBatch) {
    // phase order enforced: tile groups with K split across the waves
    const int total_k = known ? reg.total_k : 0;
    const int grid = total_k > 0 ? std::min(total_k, cus * 2) : cus * 2;
    hipLaunchKernelGGL((tcq_stack_ordered_kernel<KB, NS>), dim3(grid), dim3(kGroupThreads), 0, s, ro, plan, cb,
                       spin_limit);
  } else if (batch <= kSlotMaxBatch) {
    const int grid = (int)(total_blocks < (int64_t)cus * 2 ? total_blocks : (int64_t)cus * 2);
    PlanArgs pa = {0, 0, 0, 0};
    if (known) pa = {reg.lin_off, ordered ? reg.sched_o_off : reg.sched_u_off, reg.total, reg.batch};
    hipLaunchKernelGGL((tcq_stack_slot_kernel<KB, NS, 4>), dim3(grid), dim3(kGroupThreads), 0, s, ro, plan, cb,
                       ordered, spin_limit, pa);
  } else {
    // one 16-wave workgroup per CU (64 KiB table + two 32 KiB z chunks)
    const int grid = (int)(total_blocks < (int64_t)cus ? total_blocks : (int64_t)cus);
    const size_t zbytes = (size_t)2 * kWideChunkHalves * 2;
    if (batch <= 16) {
      auto kern = tcq_stack_wide_kernel<KB, NS, 1>;
      allow_dynamic_lds(reinterpret_cast<const void*>(kern), kTableBytes + 256);
      hipLaunchKernelGGL(kern, dim3(grid), dim3(kWideThreads), zbytes, s, ro, plan, cb, ordered, spin_limit);
    } else {
      // 17..32 rows: two row tiles per wave, 8 waves (each B operand read
      // feeds both tiles' MFMAs)
      auto kern = tcq_stack_wide_kernel<KB, NS, 2, 2>;
      allow_dynamic_lds(reinterpret_cast<const void*>(kern), kTableBytes + 256);
      hipLaunchKernelGGL(kern, dim3(grid), dim3(kWideThreads / 2), zbytes, s, ro, plan, cb, ordered, spin_limit);
    }
  }
  return launch_status();
}


// Host-side sizes of a stack (validated).
struct StackSizes {
  int n_phases;
  int64_t total_blocks, n_rot, zbuf_bytes, min_g4;
  int64_t n_rot_packed;  // rotation tiles of blocks <= 4096 (the first n_rot_packed of n_rot)
};

inline int64_t zbuf_linear_bytes(int64_t batch, int64_t G4) { return (batch * G4 * kChunkCols * 2 + 255) & ~(int64_t)255; }

inline int stack_sizes(const tp_stack_linear* linears, int n_linears, int bits, int64_t batch, StackSizes* out) {
  if (!linears) return TP_ERR_NULL_POINTER;
  if (n_linears < 1 || n_linears > kStackMaxLinears || batch < 1 || batch > 32) return TP_ERR_BAD_DIMS;
  StackSizes z = {1, 0, 0, 0, INT32_MAX, 0};
  for (int i = 0; i < n_linears; ++i) {
    const tp_stack_linear& l = linears[i];
    if (l.phase < 0 || l.phase >= kStackMaxPhases) return TP_ERR_BAD_DIMS;
    // Phases start at 0 and rise by at most 1 along the list: a phase waits
    // for the one before it only, so an empty phase in between would let the
    // phase after it start before the phase before the gap ended.
    if (i == 0 ? l.phase != 0 : (l.phase < linears[i - 1].phase || l.phase > linears[i - 1].phase + 1))
      return TP_ERR_BAD_DIMS;
    if (l.phase + 1 > z.n_phases) z.n_phases = l.phase + 1;
    Geom g;
    const int st = tiled_geom(l.n, l.d, bits, &g);
    if (st) return st;
    const int64_t blocks = (g.T + kWavesPerGroup - 1) / kWavesPerGroup;
    if (blocks >= (1 << kStackBlockBits)) return TP_ERR_BAD_DIMS;
    z.total_blocks += blocks;
    if (g.G4 < z.min_g4) z.min_g4 = g.G4;
    // (a block that is no power of 2 dividing d is refused by the plan's
    // set-up; it adds no rotation tiles here)
    const int64_t hb = l.block;
    if (hb >= 1 && !(hb & (hb - 1)) && l.d % hb == 0 && hb <= 16384) {
      const int64_t tiles = rot_tiles(batch, l.d, hb);
      z.n_rot += tiles;
      if (hb <= kRotTile) z.n_rot_packed += tiles;
    }
    z.zbuf_bytes += zbuf_linear_bytes(batch, g.G4);
  }
  // z buffer offsets are 32-bit and lanes past the batch read at 2^31: keep it below 2 GiB
  if (z.total_blocks > INT32_MAX / 2 || z.n_rot > INT32_MAX || z.zbuf_bytes >= ((int64_t)1 << 31))
    return TP_ERR_BAD_DIMS;
  *out = z;
  return TP_OK;
}

}  // namespace tp

using namespace tp;

extern "C" int64_t tp_stack_plan_bytes(const tp_stack_linear* linears, int n_linears, int bits, int64_t batch) {
  if (bits < 2 || bits > 4) return 0;
  StackSizes z;
  if (stack_sizes(linears, n_linears, bits, batch, &z) != TP_OK) return 0;
  return (int64_t)stack_layout(n_linears, z.n_phases, (int)z.total_blocks, (int)z.n_rot, z.zbuf_bytes).total;
}

extern "C" int tp_stack_plan_init(const tp_stack_linear* linears, int n_linears, int bits,
                                  int64_t batch, void* plan, int64_t plan_bytes) {
  if (!linears || !plan) return TP_ERR_NULL_POINTER;
  if (bits < 2 || bits > 4) return TP_ERR_UNSUPPORTED_BITS;
  StackSizes z;
  int st = stack_sizes(linears, n_linears, bits, batch, &z);
  if (st) return st;
  const StackLayout lay = stack_layout(n_linears, z.n_phases, (int)z.total_blocks, (int)z.n_rot, z.zbuf_bytes);
  if (plan_bytes < (int64_t)lay.total) return TP_ERR_WORKSPACE;
  if ((uintptr_t)plan & 255) return TP_ERR_MISALIGNED;
  // Everything before the z buffer is written from the host; the z buffer
  // is cleared once here (its columns past d stay zero: the rotation writes
  // only the columns of whole blocks) and every run fills the rest before
  // reading it.
  char* host = (char*)calloc(1, lay.zbuf);
  if (!host) return TP_ERR_HIP;
  StackInfo* h = reinterpret_cast<StackInfo*>(host + kStackRO);
  LinearDesc* lin = reinterpret_cast<LinearDesc*>(host + lay.lin);
  int32_t* prefix = reinterpret_cast<int32_t*>(host + lay.prefix);
  int32_t* lphase = reinterpret_cast<int32_t*>(host + lay.lphase);
  int32_t* pblocks = reinterpret_cast<int32_t*>(host + lay.pblocks);
  int32_t* sched_o = reinterpret_cast<int32_t*>(host + lay.sched_o);
  int32_t* sched_u = reinterpret_cast<int32_t*>(host + lay.sched_u);
  int32_t* sched_wo = reinterpret_cast<int32_t*>(host + lay.sched_wo);
  int32_t* sched_wu = reinterpret_cast<int32_t*>(host + lay.sched_wu);
  int32_t* ptiles = reinterpret_cast<int32_t*>(host + lay.ptiles);
  OrdBlockDesc* oblk = reinterpret_cast<OrdBlockDesc*>(host + lay.oblk);
  int64_t total_k = 0;
  RotItem* items = reinterpret_cast<RotItem*>(host + lay.rot_items);
  char* zbuf = reinterpret_cast<char*>(plan) + lay.zbuf;
  int64_t total = 0, rot_p = 0, rot_b = 0, zoff = 0;
  for (int i = 0; i < n_linears; ++i) {
    const tp_stack_linear& l = linears[i];
    Geom g;
    tiled_geom(l.n, l.d, bits, &g);  // validated by stack_sizes
    if (!l.path_tiled || !l.member_tiled || !l.x || !l.rot_scale || !l.scales || !l.y) {
      st = TP_ERR_NULL_POINTER;
      break;
    }
    const int64_t hb = l.block;
    if (hb < 1 || (hb & (hb - 1)) || l.d % hb || hb > 16384) { st = TP_ERR_BAD_BLOCK; break; }
    if (l.ldx < l.d || (l.ldx & 3) || (l.d & 3) || ((uintptr_t)l.x & 7) || ((uintptr_t)l.rot_scale & 7) ||
        ((uintptr_t)l.path_tiled & 15) || ((uintptr_t)l.member_tiled & 15)) {
      st = TP_ERR_MISALIGNED;
      break;
    }
    if (l.ldy < l.n) { st = TP_ERR_BAD_DIMS; break; }
    LinearDesc& L = lin[i];
    L.path = reinterpret_cast<const uint32_t*>(l.path_tiled);
    L.member = reinterpret_cast<const uint32_t*>(l.member_tiled);
    L.x = l.x;
    L.rs = l.rot_scale;
    L.scales = l.scales;
    L.bias = l.bias;
    L.y = l.y;
    L.ws = nullptr;
    L.cnt = nullptr;
    L.z = z.zbuf_bytes ? reinterpret_cast<uint16_t*>(zbuf + zoff) : nullptr;
    L.hdiv = (float)__builtin_sqrt((double)hb);
    L.n = (int32_t)l.n;
    L.d = (int32_t)l.d;
    L.T = (int32_t)g.T;
    L.G = (int32_t)g.G;
    L.G4 = (int32_t)g.G4;
    L.ldx = (int32_t)l.ldx;
    L.ldy = (int32_t)l.ldy;
    L.kg = (int32_t)g.G4;
    L.blocks = (int32_t)((g.T + kWavesPerGroup - 1) / kWavesPerGroup);
    L.hb = (int32_t)hb;
    prefix[i] = (int32_t)total;
    lphase[i] = l.phase;
    pblocks[l.phase] += L.blocks;
    for (int b = 0; b < L.blocks; ++b) sched_o[total + b] = (i << kStackBlockBits) | b;
    ptiles[l.phase] += L.T;
    total += L.blocks;
    if (z.zbuf_bytes) {
      const int zld = (int)g.G4 * kChunkCols;
      if (hb <= kRotTile) {
        // packed tiles over the (batch row, block) pairs; every x load is
        // range-checked against the span of the batch rows, which must stay
        // below the 2^31-byte offset of the loads past the last block
        if (((batch - 1) * l.ldx + l.d) * 2 > (int64_t)INT32_MAX) { st = TP_ERR_BAD_DIMS; break; }
        const int64_t nblk = l.d / hb, bpt = kRotTile / hb;
        const int64_t tiles = rot_tiles(batch, l.d, hb);
        for (int64_t t = 0; t < tiles; ++t) {
          RotItem& R = items[rot_p++];
          R.x = l.x;
          R.rs = l.rot_scale;
          R.z = L.z;
          R.k = (int32_t)(t * bpt);
          R.d = (int32_t)l.d;
          R.hb = (int32_t)hb;
          R.zld = zld;
          R.hdiv = L.hdiv;
          R.ldx = (int32_t)l.ldx;
          R.nblk = (int32_t)nblk;
          R.nbt = (int32_t)(batch * nblk);
          R.logh = __builtin_ctzll((unsigned long long)hb);
          R.hrecip = 1.f / L.hdiv;
        }
      } else {
        for (int64_t b = 0; b < batch; ++b) {
          for (int k = 0; k < (int)(l.d / kRotTile); ++k) {
            RotItem& R = items[z.n_rot_packed + rot_b++];
            R.x = l.x + b * l.ldx;
            R.rs = l.rot_scale;
            R.z = L.z + b * zld;
            R.k = k;
            R.d = (int32_t)l.d;
            R.hb = (int32_t)hb;
            R.zld = zld;
            R.hdiv = L.hdiv;
            R.logh = __builtin_ctzll((unsigned long long)hb);
            R.hrecip = 1.f / L.hdiv;
          }
        }
      }
      zoff += zbuf_linear_bytes(batch, g.G4);
    }
  }
  if (st == TP_OK) {
    prefix[n_linears] = (int32_t)total;
    // Unordered schedule: blocks of the longest K first (stable), so the
    // launch ends on short blocks.
    std::vector<int> order(n_linears);
    for (int i = 0; i < n_linears; ++i) order[i] = i;
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return lin[a].G4 > lin[b].G4; });
    int64_t k = 0;
    for (int i : order)
      for (int b = 0; b < lin[i].blocks; ++b) sched_u[k++] = (i << kStackBlockBits) | b;
    // Wide blocks (16 tiles) for batch 5..32, in phase order and longest K first.
    int64_t nw = 0;
    for (int i = 0; i < n_linears; ++i)
      for (int b = 0; b < (lin[i].T + kWideWaves - 1) / kWideWaves; ++b) sched_wo[nw++] = (i << kStackBlockBits) | b;
    int64_t kw = 0;
    for (int i : order)
      for (int b = 0; b < (lin[i].T + kWideWaves - 1) / kWideWaves; ++b) sched_wu[kw++] = (i << kStackBlockBits) | b;
    // Ordered-kernel blocks, phase by phase (a phase's linears are
    // consecutive), sized for the slot-kernel grid of this device.
    const int grid = 2 * device_cu_count();
    for (int i0 = 0; i0 < n_linears;) {
      int i1 = i0 + 1;
      while (i1 < n_linears && lphase[i1] == lphase[i0]) ++i1;
      total_k += ord_phase_blocks(lin, i0, i1, grid, oblk + total_k);
      i0 = i1;
    }
    h->total_wide = (int32_t)nw;
    h->total_k = (int32_t)total_k;
    h->n_lin = n_linears;
    h->total_blocks = (int32_t)total;
    h->n_phases = z.n_phases;
    h->batch = (int32_t)batch;
    h->n_rot = (int32_t)(rot_p + rot_b);
    h->n_rot_packed = (int32_t)rot_p;
    h->min_g4 = (int32_t)z.min_g4;
    h->zbuf_bytes = z.zbuf_bytes;
    if (hipMemcpy(plan, host, lay.zbuf, hipMemcpyHostToDevice) != hipSuccess) st = TP_ERR_HIP;
    else if (z.zbuf_bytes && (hipMemset(zbuf, 0, (size_t)z.zbuf_bytes) != hipSuccess ||
                              hipDeviceSynchronize() != hipSuccess))
      st = TP_ERR_HIP;
  }
  {
    std::lock_guard<std::mutex> lock(g_plan_mutex);
    if (st == TP_OK && z.n_rot > 0)
      g_plans[plan] = {(int)rot_p, (int)rot_b, (int)total, (int)batch, (int)total_k, (int64_t)(lay.lin - kStackRO),
                       (int64_t)(lay.sched_o - kStackRO), (int64_t)(lay.sched_u - kStackRO)};
    else
      g_plans.erase(plan);
  }
  free(host);
  return st;
}

extern "C" int tp_stack_rotate(void* plan, int64_t batch, void* stream) {
  if (!plan) return TP_ERR_NULL_POINTER;
  if (batch < 1 || batch > 32) return TP_ERR_BAD_DIMS;
  const char* ro = reinterpret_cast<const char*>(plan) + kStackRO;
  PlanReg reg;
  const bool known = plan_lookup(plan, &reg);
  hipStream_t s = (hipStream_t)stream;
  if (known) {
    // a few tiles per CU: one latency chain, the permlane butterflies; more
    // (batch 32: 7488 tiles at Qwen3-4B): VALU issue, the bpermute ones
    // (batch-32 step 510.1 -> 508.8 us against the permlane ones)
    const bool swap = (int64_t)reg.n_rot_packed + reg.n_rot_big <= 4 * (int64_t)device_cu_count();
    if (reg.n_rot_packed > 0) {
      if (swap)
        hipLaunchKernelGGL((tcq_stack_rotate_kernel<true, true>), dim3(reg.n_rot_packed), dim3(kRotThreads), 0, s, ro);
      else
        hipLaunchKernelGGL((tcq_stack_rotate_kernel<true, false>), dim3(reg.n_rot_packed), dim3(kRotThreads), 0, s, ro);
    }
    if (reg.n_rot_big > 0) {
      if (swap)
        hipLaunchKernelGGL((tcq_stack_rotate_big_kernel<true, true>), dim3(reg.n_rot_big), dim3(kRotThreads), 0, s, ro);
      else
        hipLaunchKernelGGL((tcq_stack_rotate_big_kernel<true, false>), dim3(reg.n_rot_big), dim3(kRotThreads), 0, s, ro);
    }
  } else {
    const int grid = 2 * device_cu_count();
    hipLaunchKernelGGL((tcq_stack_rotate_kernel<false, false>), dim3(grid), dim3(kRotThreads), 0, s, ro);
    hipLaunchKernelGGL((tcq_stack_rotate_big_kernel<false, false>), dim3(grid), dim3(kRotThreads), 0, s, ro);
  }
  return launch_status();
}

extern "C" int tp_stack_gemv(void* plan, int64_t batch, const uint16_t* codebook, int bits,
                             int n_states, int ordered, int64_t total_blocks, void* stream) {
  if (!plan || !codebook) return TP_ERR_NULL_POINTER;
  if ((uintptr_t)codebook & 3) return TP_ERR_MISALIGNED;  // read as dwords through the scalar cache
  if (total_blocks < 1 || total_blocks > INT32_MAX) return TP_ERR_BAD_DIMS;
  if (batch < 1 || batch > 32) return TP_ERR_BAD_DIMS;
  const int spin_limit = 1 << 22;  // ~ seconds of s_sleep polling; ends the wait regardless
  char* p = reinterpret_cast<char*>(plan);
  hipStream_t s = (hipStream_t)stream;
  switch (bits * 100 + n_states) {
    case 204: return launch_gemv<2, 4>(p, total_blocks, batch, codebook, ordered, spin_limit, s);
    case 208: return launch_gemv<2, 8>(p, total_blocks, batch, codebook, ordered, spin_limit, s);
    case 216: return launch_gemv<2, 16>(p, total_blocks, batch, codebook, ordered, spin_limit, s);
    case 264: return launch_gemv<2, 64>(p, total_blocks, batch, codebook, ordered, spin_limit, s);
    case 304: return launch_gemv<3, 4>(p, total_blocks, batch, codebook, ordered, spin_limit, s);
    case 308: return launch_gemv<3, 8>(p, total_blocks, batch, codebook, ordered, spin_limit, s);
    case 316: return launch_gemv<3, 16>(p, total_blocks, batch, codebook, ordered, spin_limit, s);
    case 364: return launch_gemv<3, 64>(p, total_blocks, batch, codebook, ordered, spin_limit, s);
    case 404: return launch_gemv<4, 4>(p, total_blocks, batch, codebook, ordered, spin_limit, s);
    case 408: return launch_gemv<4, 8>(p, total_blocks, batch, codebook, ordered, spin_limit, s);
    case 416: return launch_gemv<4, 16>(p, total_blocks, batch, codebook, ordered, spin_limit, s);
    case 464: return launch_gemv<4, 64>(p, total_blocks, batch, codebook, ordered, spin_limit, s);
    default: return TP_ERR_UNSUPPORTED_STATES;
  }
}

extern "C" int tp_stack_run(void* plan, int64_t batch, const uint16_t* codebook, int bits,
                            int n_states, int ordered, int64_t total_blocks, void* stream) {
  if (!plan || !codebook) return TP_ERR_NULL_POINTER;
  if (total_blocks < 1 || total_blocks > INT32_MAX) return TP_ERR_BAD_DIMS;
  if (bits < 2 || bits > 4) return TP_ERR_UNSUPPORTED_BITS;
  if (n_states != 4 && n_states != 8 && n_states != 16 && n_states != 64) return TP_ERR_UNSUPPORTED_STATES;
  // (every check of tp_stack_gemv before the rotation launch rewrites z)
  if ((uintptr_t)codebook & 3) return TP_ERR_MISALIGNED;
  const int st = tp_stack_rotate(plan, batch, stream);
  if (st) return st;
  return tp_stack_gemv(plan, batch, codebook, bits, n_states, ordered, total_blocks, stream);
}

extern "C" int64_t tp_stack_plan_blocks(const int64_t* ns, int n_linears) {
  if (!ns || n_linears < 1) return 0;
  int64_t total = 0;
  for (int i = 0; i < n_linears; ++i) {
    if (ns[i] <= 0) return 0;
    const int64_t T = (ns[i] + kTileRows - 1) / kTileRows;
    total += (T + kWavesPerGroup - 1) / kWavesPerGroup;
  }
  return total;
}

extern "C" int tp_stack_error(const void* plan, int* error_out) {
  if (!plan || !error_out) return TP_ERR_NULL_POINTER;
  StackCounters h;
  if (hipMemcpy(&h, plan, sizeof(h), hipMemcpyDeviceToHost) != hipSuccess) return TP_ERR_HIP;
  *error_out = (int)h.error;
  return TP_OK;
}
