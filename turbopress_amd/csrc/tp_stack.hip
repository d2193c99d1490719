// One persistent launch for every packed linear of a decode step.
//
// The reference runs a decode step as one graph node pair per projection
// (turbopress/runtime.py:312-316 inside the HF decoder, replayed by
// scripts/graph_decode_bench.py:103-115).  On MI355X a kernel launch inside a
// graph costs ~1.5 us and a 9.4 MB GEMV cannot reach HBM speed before its
// latency chain ends, so here one launch streams the whole list of linears:
//
//   * work = "blocks" of 8 row tiles x the full K range of one linear, handed
//     to persistent workgroups by an atomic ticket (self-resetting);
//   * a block walks K in chunks of 2 units (512 columns): per chunk the
//     workgroup rotates its slice of x into LDS (tp_tiled_common.h,
//     stage_z*), every wave decodes and multiplies its tile's units, and the
//     loads of the next chunk are already in flight;
//   * full-K blocks need no split-K reduction: each wave writes its 16 rows;
//   * optional phase ordering: linears carry a phase index and, when
//     `ordered` is set, a block of phase p starts only after every block of
//     phase p-1 has finished (bounded wait; on timeout the plan's error flag
//     is set and the block proceeds, so the kernel always terminates).
#include "tp_tiled_common.h"

namespace tp {

constexpr int kStackMaxPhases = 4096;

// Plan layout (device memory):
//   [0, 64)            StackCounters  -- written by the kernel (atomics)
//   [64, ...)          StackInfo, LinearDesc[n_lin], prefix[n_lin+1],
//                      lphase[n_lin], pblocks[n_phases]  -- read-only
//   [pdone offset, ..) pdone[n_phases] -- written by the kernel (atomics)
// The read-only part is passed as a separate const __restrict__ argument so
// its loads go through the scalar cache into SGPRs.
struct StackCounters {
  uint32_t ticket;   // next block index (reset to 0 by the last workgroup out)
  uint32_t exited;   // workgroups past the loop (reset likewise)
  uint32_t error;    // 1: a phase wait timed out; 2: launched for fewer batch rows than the plan
  uint32_t reserved[13];
};

struct StackInfo {
  int32_t n_lin;
  int32_t total_blocks;
  int32_t n_phases;
  int32_t batch;
  int64_t pdone_offset;   // byte offset of pdone from the plan start
  int64_t reserved;
};

struct StackRO {  // views into the read-only part
  const StackInfo* info;
  const LinearDesc* lin;
  const int32_t* prefix;   // [n_lin + 1] first block of each linear
  const int32_t* lphase;   // [n_lin]
  const int32_t* pblocks;  // [n_phases] blocks per phase
};

constexpr size_t kStackRO = sizeof(StackCounters);

__host__ __device__ inline size_t stack_plan_offsets(int n_lin, int n_phases, size_t* o_lin, size_t* o_prefix,
                                                     size_t* o_lphase, size_t* o_pblocks, size_t* o_pdone) {
  size_t o = kStackRO + sizeof(StackInfo);
  *o_lin = o;
  o += sizeof(LinearDesc) * (size_t)n_lin;
  *o_prefix = o;
  o += sizeof(int32_t) * (size_t)(n_lin + 1);
  *o_lphase = o;
  o += sizeof(int32_t) * (size_t)n_lin;
  *o_pblocks = o;
  o += sizeof(int32_t) * (size_t)n_phases;
  o = (o + 63) & ~(size_t)63;
  *o_pdone = o;
  o += sizeof(uint32_t) * (size_t)n_phases;
  return (o + 255) & ~(size_t)255;
}

// `ro` points at plan + kStackRO.
__device__ inline StackRO stack_ro(const char* __restrict__ ro) {
  const StackInfo* info = reinterpret_cast<const StackInfo*>(ro);
  size_t a, b, c, d, e;
  stack_plan_offsets(info->n_lin, info->n_phases, &a, &b, &c, &d, &e);
  StackRO v;
  v.info = info;
  v.lin = reinterpret_cast<const LinearDesc*>(ro + (a - kStackRO));
  v.prefix = reinterpret_cast<const int32_t*>(ro + (b - kStackRO));
  v.lphase = reinterpret_cast<const int32_t*>(ro + (c - kStackRO));
  v.pblocks = reinterpret_cast<const int32_t*>(ro + (d - kStackRO));
  return v;
}

// Path/member words of one chunk (kMaxUnitsPerBlock units) of one lane.
template <int MW>
struct ChunkRegs {
  uint2 X[kMaxUnitsPerBlock];
  uint32_t M[kMaxUnitsPerBlock][MW];
};

template <int MW>
__device__ __forceinline__ ChunkRegs<MW> load_chunk(const LinearDesc& L, const uint32_t* pt, const uint32_t* mt,
                                                     int ch, bool active, int q, int r) {
  // Branch-free: units past the block's K range (and inactive waves, whose
  // pointers address tile 0) reload unit 0 of the chunk; they are never used.
  ChunkRegs<MW> c;
  const int gu0 = ch * kMaxUnitsPerBlock;
  const int ngu = min(kMaxUnitsPerBlock, L.G4 - gu0);
  (void)active;
#pragma unroll
  for (int u = 0; u < kMaxUnitsPerBlock; ++u) {
    const int g = 4 * (gu0 + (u < ngu ? u : 0)) + q;
    c.X[u] = gld2(pt + (g * kTileRows + r) * 2);
#pragma unroll
    for (int i = 0; i < MW; ++i) c.M[u][i] = gld(mt + (g * kTileRows + r) * MW + i);
  }
  return c;
}

template <int KB, int NS, int NBT>
__global__ void __launch_bounds__(kGroupThreads) __attribute__((amdgpu_waves_per_eu(NBT == 1 ? 4 : 2)))
tcq_stack_kernel(const char* __restrict__ plan_ro, char* __restrict__ plan_rw,
                 const uint16_t* __restrict__ codebook, int ordered, int spin_limit, int zrows) {
  __shared__ __attribute__((aligned(16))) uint32_t table[kTableWords];
  extern __shared__ __attribute__((aligned(16))) uint16_t zl[];
  __shared__ int s_next;
  constexpr int MW = member_words(KB);
  // Sizes come from the plan itself, never from the caller.
  const StackRO P = stack_ro(plan_ro);
  const int n_lin = P.info->n_lin;
  const int n_phases = P.info->n_phases;
  const int batch = P.info->batch;
  const int total = P.info->total_blocks;
  StackCounters* C = reinterpret_cast<StackCounters*>(plan_rw);
  uint32_t* pdone = reinterpret_cast<uint32_t*>(plan_rw + P.info->pdone_offset);
  if (batch > 16 * NBT || batch > zrows) {  // staged z rows would not fit: refuse uniformly
    if (threadIdx.x == 0 && blockIdx.x == 0) atomicExch(&C->error, 2u);
    return;
  }
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r = lane & 15;
  const int q = lane >> 4;
  const uint32_t laneoff = (uint32_t)lane << 2;
  const uint32_t cb_lane = gld(codebook + (lane & ((2 << KB) - 1)));

  if (tid == 0) s_next = (int)atomicAdd(&C->ticket, 1u);
  build_pair_table_lanes<KB>(table, cb_lane, tid, kGroupThreads);
  __syncthreads();
  // The ticket travels through LDS; make its uniformity explicit so that the
  // descriptor reads below become scalar loads (vector loads would be followed
  // by waits that also drain the weight prefetches in flight).
  int blk = __builtin_amdgcn_readfirstlane(s_next);

  while (blk < total) {
    // Linear of this block: last li with prefix[li] <= blk (uniform).
    int lo = 0, hi = n_lin - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (P.prefix[mid] <= blk) lo = mid; else hi = mid - 1;
    }
    const int li = __builtin_amdgcn_readfirstlane(lo);
    const LinearDesc L = P.lin[li];  // copied to registers once per block
    const int t = (blk - P.prefix[li]) * kWavesPerGroup + wave;
    const bool active = t < L.T;
    const int nch = (L.G4 + kMaxUnitsPerBlock - 1) / kMaxUnitsPerBlock;
    const uint32_t* pt = L.path + (size_t)(active ? t : 0) * L.G * (kTileRows * 2);
    const uint32_t* mt = L.member + (size_t)(active ? t : 0) * L.G * (kTileRows * MW);

    // Claim the next block now; its index is needed only after this one.
    uint32_t next_ticket = 0;
    if (tid == 0) next_ticket = atomicAdd(&C->ticket, 1u);

    if (ordered) {
      const int ph = P.lphase[li];
      if (ph > 0) {
        if (tid == 0) {
          const uint32_t need = (uint32_t)P.pblocks[ph - 1];
          int spins = 0;
          while (__hip_atomic_load(&pdone[ph - 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < need) {
            if (++spins > spin_limit) {
              atomicExch(&C->error, 1u);
              break;
            }
            __builtin_amdgcn_s_sleep(8);
          }
        }
        __syncthreads();
      }
    }

    // Chunks run ping-pong over two register sets (A, B): a set is refilled
    // only after its last use, so the prefetched values never need a register
    // copy (a copy would have to wait for the prefetch to land).
    uint32_t x1_last = 0;
    float4_t acc[NBT];
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt) acc[bt] = float4_t{0.f, 0.f, 0.f, 0.f};
    auto chunk_body = [&](int ch, const ChunkRegs<MW>& regs, const ZPrefetch& zpf) {
      const int gu0 = ch * kMaxUnitsPerBlock;
      const int ngu = min(kMaxUnitsPerBlock, L.G4 - gu0);
      const bool small = ngu * batch <= kWavesPerGroup && L.hb <= 2 * kChunkCols;
      __syncthreads();  // z of the previous chunk is no longer read
      if (small) {
        if (zpf.valid) stage_z_prefetched<true>(L, gu0, batch, zl, wave, lane, zpf);
      } else {
        stage_z<true>(L, gu0, ngu, batch, zl, wave, lane);
      }
      __syncthreads();
      if (active) {
#pragma unroll
        for (int u = 0; u < kMaxUnitsPerBlock; ++u) {
          if (u >= ngu) break;
          const int gu = gu0 + u;
          process_unit<KB, NS, NBT>(regs.X[u], regs.M[u], x1_last, gu, (4 * gu + q - 4 * gu0) * kSegCols, q, r,
                                    lane, laneoff, table, zl, batch, acc);
          x1_last = regs.X[u].y;
        }
      }
    };
    auto ngu_of = [&](int ch) { return ch < nch ? min(kMaxUnitsPerBlock, L.G4 - ch * kMaxUnitsPerBlock) : 0; };
    ChunkRegs<MW> ra = load_chunk<MW>(L, pt, mt, 0, active, q, r);
    ZPrefetch za = prefetch_z<true>(L, 0, ngu_of(0), batch, wave, lane);
    for (int ch = 0; ch < nch; ch += 2) {
      const ChunkRegs<MW> rb = load_chunk<MW>(L, pt, mt, ch + 1 < nch ? ch + 1 : ch, active && ch + 1 < nch, q, r);
      const ZPrefetch zb = prefetch_z<true>(L, (ch + 1) * kMaxUnitsPerBlock, ngu_of(ch + 1), batch, wave, lane);
      chunk_body(ch, ra, za);
      if (ch + 1 >= nch) break;
      ra = load_chunk<MW>(L, pt, mt, ch + 2 < nch ? ch + 2 : ch, active && ch + 2 < nch, q, r);
      za = prefetch_z<true>(L, (ch + 2) * kMaxUnitsPerBlock, ngu_of(ch + 2), batch, wave, lane);
      chunk_body(ch + 1, rb, zb);
    }

    // Full-K epilogue: lane holds rows 4q..4q+3 of its tile for batch column r.
    if (active) {
      const int row0 = t * kTileRows + 4 * q;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = row0 + i;
        if (row >= L.n) continue;
        const float sc = h2f(gld(L.scales + row));
        const float bs = L.bias ? h2f(gld(L.bias + row)) : 0.f;
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) {
          const int nb = bt * 16 + r;
          if (nb >= batch) continue;
          uint16_t out = f2h(acc[bt][i] * sc);
          if (L.bias) out = f2h(h2f(out) + bs);
          gst(L.y + (size_t)nb * L.ldy + row, out);
        }
      }
    }
    if (ordered) {
      __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (tid == 0) atomicAdd(&pdone[P.lphase[li]], 1u);
    }
    if (tid == 0) s_next = (int)next_ticket;
    __syncthreads();
    blk = __builtin_amdgcn_readfirstlane(s_next);
  }

  // The last workgroup out resets the counters for the next launch.
  if (tid == 0) {
    const uint32_t e = atomicAdd(&C->exited, 1u);
    if (e == gridDim.x - 1) {
      for (int p = 0; p < n_phases; ++p) atomicExch(&pdone[p], 0u);
      atomicExch(&C->ticket, 0u);
      atomicExch(&C->exited, 0u);
    }
  }
}

// z staging rows: 8 for batch <= 8 keeps table + z + ticket slot within half
// of the 160 KiB LDS, so two workgroups share a CU.
inline int stack_z_rows(int64_t batch) { return batch <= 8 ? 8 : batch <= 16 ? 16 : 32; }

template <int KB, int NS, int NBT>
void launch_stack(char* plan, int grid, int64_t batch, const uint16_t* cb, int ordered, int spin_limit,
                  hipStream_t s) {
  hipLaunchKernelGGL((tcq_stack_kernel<KB, NS, NBT>), dim3(grid), dim3(kGroupThreads),
                     (size_t)stack_z_rows(batch) * kZCols * 2, s, (const char*)(plan + kStackRO), plan, cb,
                     ordered, spin_limit, stack_z_rows(batch));
}

}  // namespace tp

using namespace tp;

extern "C" int64_t tp_stack_plan_bytes(int n_linears, int n_phases) {
  if (n_linears < 1 || n_phases < 1 || n_phases > kStackMaxPhases) return 0;
  size_t a, b, c, d, e;
  return (int64_t)stack_plan_offsets(n_linears, n_phases, &a, &b, &c, &d, &e);
}

extern "C" int tp_stack_plan_init(const tp_stack_linear* linears, int n_linears, int bits,
                                  int64_t batch, void* plan, int64_t plan_bytes) {
  if (!linears || !plan) return TP_ERR_NULL_POINTER;
  if (n_linears < 1 || batch < 1 || batch > 32) return TP_ERR_BAD_DIMS;
  if (bits != 2 && bits != 3) return TP_ERR_UNSUPPORTED_BITS;
  int n_phases = 1;
  for (int i = 0; i < n_linears; ++i) {
    if (linears[i].phase < 0 || linears[i].phase >= kStackMaxPhases) return TP_ERR_BAD_DIMS;
    if (i > 0 && linears[i].phase < linears[i - 1].phase) return TP_ERR_BAD_DIMS;  // phases ascend
    if (linears[i].phase + 1 > n_phases) n_phases = linears[i].phase + 1;
  }
  size_t o_lin, o_prefix, o_lphase, o_pdone, o_pblocks;
  const size_t need = stack_plan_offsets(n_linears, n_phases, &o_lin, &o_prefix, &o_lphase, &o_pblocks, &o_pdone);
  if (plan_bytes < (int64_t)need) return TP_ERR_WORKSPACE;
  if ((uintptr_t)plan & 255) return TP_ERR_MISALIGNED;
  char* host = (char*)calloc(1, need);
  if (!host) return TP_ERR_HIP;
  StackInfo* h = reinterpret_cast<StackInfo*>(host + kStackRO);
  LinearDesc* lin = reinterpret_cast<LinearDesc*>(host + o_lin);
  int32_t* prefix = reinterpret_cast<int32_t*>(host + o_prefix);
  int32_t* lphase = reinterpret_cast<int32_t*>(host + o_lphase);
  int32_t* pblocks = reinterpret_cast<int32_t*>(host + o_pblocks);
  int64_t total = 0;
  int st = TP_OK;
  for (int i = 0; i < n_linears && st == TP_OK; ++i) {
    const tp_stack_linear& l = linears[i];
    Geom g;
    st = tiled_geom(l.n, l.d, bits, &g);
    if (st) break;
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
    total += L.blocks;
  }
  if (st == TP_OK && total > INT32_MAX) st = TP_ERR_BAD_DIMS;
  if (st == TP_OK) {
    prefix[n_linears] = (int32_t)total;
    h->n_lin = n_linears;
    h->total_blocks = (int32_t)total;
    h->n_phases = n_phases;
    h->batch = (int32_t)batch;
    h->pdone_offset = (int64_t)o_pdone;
    if (hipMemcpy(plan, host, need, hipMemcpyHostToDevice) != hipSuccess) st = TP_ERR_HIP;
  }
  free(host);
  return st;
}

extern "C" int tp_stack_run(void* plan, int64_t batch, const uint16_t* codebook, int bits,
                            int n_states, int ordered, int64_t total_blocks, void* stream) {
  if (!plan || !codebook) return TP_ERR_NULL_POINTER;
  if (total_blocks < 1 || total_blocks > INT32_MAX) return TP_ERR_BAD_DIMS;
  if (batch < 1 || batch > 32) return TP_ERR_BAD_DIMS;
  const int nbt = batch <= 16 ? 1 : 2;
  const int cus = device_cu_count();
  const int per_cu = batch <= 8 ? 2 : 1;
  const int grid = (int)(total_blocks < (int64_t)cus * per_cu ? total_blocks : (int64_t)cus * per_cu);
  const int spin_limit = 1 << 22;  // ~ seconds of s_sleep polling; ends the wait regardless
  char* p = reinterpret_cast<char*>(plan);
  hipStream_t s = (hipStream_t)stream;
#define TP_STACK(KB, NS)                                                       \
  (nbt == 1 ? launch_stack<KB, NS, 1>(p, grid, batch, codebook, ordered, spin_limit, s) \
            : launch_stack<KB, NS, 2>(p, grid, batch, codebook, ordered, spin_limit, s))
  switch (bits * 100 + n_states) {
    case 204: TP_STACK(2, 4); break;
    case 208: TP_STACK(2, 8); break;
    case 216: TP_STACK(2, 16); break;
    case 264: TP_STACK(2, 64); break;
    case 304: TP_STACK(3, 4); break;
    case 308: TP_STACK(3, 8); break;
    case 316: TP_STACK(3, 16); break;
    case 364: TP_STACK(3, 64); break;
    default: return TP_ERR_UNSUPPORTED_STATES;
  }
#undef TP_STACK
  return launch_status();
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
