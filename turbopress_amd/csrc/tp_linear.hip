// One-pass decode-GEMV of one packed linear (or of 2..4 linears sharing one
// input) at batch <= 8: the operator path of PackedTCQLinear.forward
// (turbopress/runtime.py:304-334 -> triton_kernel.py:235-260 fwht_scale +
// :132-157 packed_gemv), for calls that run one projection at a time.
//
// A single 9.4 MB linear has only ~1.5 units of work per wave of the chip, so
// the launch is built around latency rather than streaming:
//   * one workgroup of 16 waves per CU; the group owns `tpw` row tiles and
//     splits each tile's K range into `s` chunks of at most 3 units (4
//     when several linears share the launch), one
//     chunk per wave, so every weight load of the launch is issued in the
//     first few hundred cycles;
//   * while those loads are in flight the workgroup builds the pair table
//     and rotates the whole input into LDS (z = blockFWHT(x * rot_scale) /
//     sqrt(block), fp32, rounded to fp16 once): every chunk then reads its B
//     operands from LDS, and no second launch or global z buffer is needed;
//   * the chunks of a tile are summed through LDS (no atomics, no workspace)
//     and chunk 0's wave writes y = fp16(sum * scale) (+ bias).
//   * K-split (one linear, Hadamard blocks <= 512 columns): for shapes whose
//     K range is long against their rows (down_proj: 160 row tiles x 38
//     units), the K range is also cut into `kparts` parts of whole Hadamard
//     blocks, one workgroup per (tile group, part), so that each workgroup
//     stages and rotates only its part of the input and every CU gets work.
//     A part's sum is stored with coherent (L2-bypassing) stores into its
//     own slice of the caller's workspace; the last part to arrive at the
//     tile's counter adds the slices in part order (a fixed order: the
//     result does not depend on which workgroup finishes last), writes y,
//     and leaves slices and counter zero.
// The per-unit decode and MFMA step is the stack kernel's (tp_slot.h).
#include "tp_slot.h"
#include "tp_rotate_tile.h"

namespace tp {

constexpr int kLinWaves = 16;
constexpr int kLinThreads = 64 * kLinWaves;

// x / d and x % d for wave-uniform 0 <= x < 8 d, d >= 1 (a batch row or a
// wave's tile: a launch holds at most 8 batch rows): at most 7 scalar
// subtractions, where a division is ~25 dependent instructions (a vector
// reciprocal and its read-back) on the way to the first weight load.
__device__ __forceinline__ int udiv_small(int x, int d, int* rem) {
  int q = 0;
  for (int i = 0; i < 7 && x >= d; ++i) {
    x -= d;
    ++q;
  }
  *rem = x;
  return q;
}
// x / d for wave-uniform x >= 0 with x * d < 2^32: one scalar multiply-high
// by m = ceil(2^32 / d), which the host computes (lin_recip; m = 0 stands for
// d = 1).  With x = q d + r, x m / 2^32 = q + r / d + x e / (d 2^32) for some
// 0 <= e < d, and x e / (d 2^32) < x / 2^32 < 1 / d, so the floor is q.
__device__ __forceinline__ int udiv_recip(int x, uint32_t m) {
  return m ? (int)__umulhi((uint32_t)x, m) : x;
}
__host__ __device__ constexpr uint32_t lin_recip(int64_t d) {
  return d <= 1 ? 0u : (uint32_t)(((int64_t)1 << 32) / d + (((int64_t)1 << 32) % d != 0));
}

// Units per wave, all loaded up front: 3, and 4 in launches of several
// linears, where it lets two 9728-row linears (gate/up sharing their input)
// fit one round of 244 workgroups (3 units: 304 workgroups on 256 CUs, two
// rounds; 17.0 -> 10.7 us at batch 1).  The single-linear variants keep 3:
// a fourth register set of loads, issued out of range when unused, made
// them ~0.3 us slower.
constexpr int kLinMaxUnits = 3;
constexpr int kLinMaxUnitsMulti = 4;
__host__ __device__ constexpr int lin_max_units(bool multi) { return multi ? kLinMaxUnitsMulti : kLinMaxUnits; }
constexpr int kLinMaxParts = kMaxInlineLinears;
constexpr int kLinRedBytes = kLinWaves * 64 * 16;    // one float4 per lane and wave
// K-split: a part's sums of one row tile are [16 rows][8 batch columns] fp32
// (512 bytes); at most kLinMaxTileParts (row tile, part) slices per call.
constexpr int kLinSliceFloats = kTileRows * 8;
constexpr int kLinMaxTileParts = 2048;
constexpr int kLinMaxKParts = 16;    // (one register per part in the reduction)
// Cache policy of buffer accesses that must be coherent across the chip's
// L2s (sc1, as agent-scope atomic loads and stores compile to).
constexpr int kCoherent = 16;

struct LinPart {
  const uint32_t* path;      // tiled path words [T][G][16][2]
  const uint32_t* member;    // tiled member words [T][G][16][MW]
  const uint16_t* x;         // first batch row of this launch
  const uint16_t* rs;        // rot_scale [d]; null: x is z already (G4 * 256 columns, zero past d)
  const uint16_t* scales;    // [n]
  const uint16_t* bias;      // [n] or null
  uint16_t* y;               // first batch row of this launch
  int32_t n, T, ldx, ldy;
  int32_t g0;                // first tile group of this linear
  int32_t reserved;
};

// Every field a wave reads at its entry comes first, then part[0]: the
// prologue's argument loads are then a few wide scalar loads of one span
// instead of one per scattered field (each wave of a 16-wave workgroup makes
// them, through one scalar cache).
struct LinArgs {
  const uint16_t* codebook;
  int32_t d, G4, hb, batch;  // batch: rows of this launch (<= SB)
  int32_t c, s, tpw;         // units per chunk, chunks per tile, tiles per group
  int32_t zstride;           // halves per staged z row (units staged * 256 + 8: rows start 4 banks apart)
  float hdiv;                // sqrt(hb)
  int32_t kparts, pu;        // K parts per tile group (1: no split), units per part
  int32_t n_part, groups;    // tile groups over all linears
  int32_t g0[kLinMaxParts];  // part[i].g0: first tile group of each linear
  uint32_t r_s, r_kparts;    // lin_recip(s), lin_recip(kparts)
  uint32_t r_pu, r_pu_last;  // lin_recip of a K part's units: every part but the last, the last (or only) part
  uint32_t r_batch;          // lin_recip(batch)
  int32_t sk, sk_last;       // chunks of c units in a K part: every part but the last, the last (or only) part
  float hrecip;              // fp32(1 / hdiv), correctly rounded
  LinPart part[kLinMaxParts];
  float* kws;                // K-split slices [kparts][T][16 rows][8] fp32 (zero between calls)
  uint32_t* kcnt;            // K-split arrival counter per row tile (zero between calls)
};
static_assert(sizeof(LinPart) == 80 && __builtin_offsetof(LinArgs, part) == 112,
              "entry fields in the first 112 bytes, then part[0]");

// Butterflies of one chunk (four columns per lane, lane-major) up to
// distance hmax / 2.  FULL: hmax = 256, every stage (no stage test: each
// test is a few scalar instructions per staged chunk, and the 16 waves of a
// workgroup share one scalar unit).
template <bool FULL>
__device__ __forceinline__ void lin_chunk_stages(int hmax, int lane, float v[4]) {
  if (FULL || hmax > 1) {
    float p = v[0], q = v[1];
    v[0] = p + q; v[1] = p - q;
    p = v[2]; q = v[3];
    v[2] = p + q; v[3] = p - q;
  }
  if (FULL || hmax > 2) {
    float p = v[0], q = v[2];
    v[0] = p + q; v[2] = p - q;
    p = v[1]; q = v[3];
    v[1] = p + q; v[3] = p - q;
  }
  // (the upper lane of a pair keeps p - v: one FMA with the lane's sign)
#pragma unroll
  for (int sft = 0; sft < 6; ++sft) {
    if (FULL || (4 << sft) < hmax) {
      const float sg = ((lane >> sft) & 1) ? -1.f : 1.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (sft == 4) v[e] = lane_swap_butterfly<4>(v[e], sg);
        else if (sft == 5) v[e] = lane_swap_butterfly<5>(v[e], sg);
        else v[e] = __builtin_fmaf(sg, v[e], lane_xor_row(v[e], 1 << sft));
      }
    }
  }
}

// Butterflies of one chunk up to distance min(hb, 256) / 2, then / sqrt(hb).
__device__ __forceinline__ void lin_chunk_fwht(const LinArgs& a, int lane, float v[4]) {
  if (a.hb >= kChunkCols) lin_chunk_stages<true>(kChunkCols, lane, v);
  else lin_chunk_stages<false>(a.hb, lane, v);
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = div_by_block_root_fx(v[e], a.hdiv, a.hrecip);
}

// z of one 256-column chunk of batch row b for Hadamard blocks <= 512, four
// columns per lane: x * rs, (hb = 512: the signed sum of the block's two
// chunks, i.e. the H_2 factor of H_512 = H_2 (x) H_256), the butterflies
// inside the chunk, then / sqrt(hb).  Columns past d are zero.
__device__ void lin_rotate_chunk(const LinArgs& a, const LinPart& P, int b, int cs, int lane, float v[4]) {
  const uint16_t* xr = P.x + (size_t)b * P.ldx;
  // v = 0 + (+-x rs) + ...: each product of two fp16 values is exact in fp32,
  // so fma(x, +-rs, v) rounds as the add does (one v_fma_mix_f32 from the
  // fp16 halves; the sign of a term is the sign bit of its rs halves).  The
  // +0 start sits in an opaque register: a literal one lets the compiler
  // split the first fma into converts and a product.
  float pz = 0.f;
  __asm__("" : "+v"(pz));
  v[0] = v[1] = v[2] = v[3] = pz;
  // (hb is a power of two: masks and shifts)
  const int nsub = a.hb > kChunkCols ? a.hb >> 8 : 1;
  const int base = a.hb > kChunkCols ? cs & ~(a.hb - 1) : cs;
  const int o = a.hb > kChunkCols ? (cs & (a.hb - 1)) >> 8 : 0;
  for (int i = 0; i < nsub; ++i) {
    const int c0 = base + i * kChunkCols + lane * 4;
    if (c0 < a.d) {  // d is a multiple of 4: a lane's group is wholly inside or outside
      const uint2 xw = gld2(xr + c0), rw = gld2(P.rs + c0);
      const uint32_t sgn = (__popc(i & o) & 1) ? 0x80008000u : 0u;
      const uint32_t r0 = rw.x ^ sgn, r1 = rw.y ^ sgn;
      v[0] = __builtin_fmaf(hlo(xw.x), hlo(r0), v[0]);
      v[1] = __builtin_fmaf(hhi(xw.x), hhi(r0), v[1]);
      v[2] = __builtin_fmaf(hlo(xw.y), hlo(r1), v[2]);
      v[3] = __builtin_fmaf(hhi(xw.y), hhi(r1), v[3]);
    }
  }
  lin_chunk_fwht(a, lane, v);
}

// Activations of the first kLinPre staging items of a wave (item wave + 16k),
// loaded at kernel start so that their latency overlaps the weight loads.
// Blocks <= 512: item = (batch row, chunk), with the other chunk of a
// 512-block; larger blocks: the chunks of batch row 0 (the first pass).
constexpr int kLinPre = 2;
// (k=4 keeps one: its member words take the registers of the other)
__host__ __device__ constexpr int lin_pre(int bits) { return bits == 4 ? 1 : kLinPre; }
template <int NPRE>
struct XPre {
  u32x2_t x[NPRE][2], r[NPRE][2];
};

// Items of the K part [pu0, pu0 + npu) (units = 256-column chunks).
template <int NPRE>
__device__ __forceinline__ XPre<NPRE> lin_prefetch_x(const LinArgs& a, const LinPart& P, int pu0, int npu,
                                                     uint32_t rnpu, int wave, int lane) {
  XPre<NPRE> f;
  const __amdgpu_buffer_rsrc_t xrs = buffer_rsrc(P.x, (uint32_t)((a.batch - 1) * P.ldx + a.d) * 2u);
  const __amdgpu_buffer_rsrc_t rrs = buffer_rsrc(P.rs, (uint32_t)a.d * 2u);
  const bool small = a.hb <= 2 * kChunkCols;
  const bool pair = small && a.hb > kChunkCols;  // a 512-block: both of its chunks
  const int items = (small ? a.batch : 1) * npu;
  // (items past the count, and the second chunk unless pair, are not loaded
  // at all -- wave-uniform branches: out-of-range loads still take their
  // turn in the workgroup's vector memory path, which the 16 waves' prologue
  // loads queue on; the staging reads only the items it loaded)
#pragma unroll
  for (int k = 0; k < NPRE; ++k) {
    const int it = wave + kLinWaves * k;
    if (it < items) {
      const int b = udiv_recip(it, rnpu);  // (it < batch * npu)
      const int ci = it - b * npu;
      const int cs = (pu0 + ci) * kChunkCols;
      const int base = pair ? cs & ~(a.hb - 1) : cs;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        if (i == 0 || pair) {
          const int c0 = base + i * kChunkCols + lane * 4;
          const bool in = c0 < a.d;
          f.x[k][i] = __builtin_amdgcn_raw_buffer_load_b64(xrs, in ? (uint32_t)(b * P.ldx + c0) * 2u : kOutOfRange, 0, 0);
          f.r[k][i] = __builtin_amdgcn_raw_buffer_load_b64(rrs, in ? (uint32_t)c0 * 2u : kOutOfRange, 0, 0);
        } else {
          f.x[k][i] = u32x2_t{0u, 0u};
          f.r[k][i] = u32x2_t{0u, 0u};
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        f.x[k][i] = u32x2_t{0u, 0u};
        f.r[k][i] = u32x2_t{0u, 0u};
      }
    }
  }
  return f;
}

// x * rs of prefetched item k (the signed sum of both chunks of a 512-block).
template <int NPRE>
__device__ __forceinline__ void lin_pre_product(const LinArgs& a, const XPre<NPRE>& f, int k, int cs, float v[4]) {
  // as lin_rotate_chunk: v = 0 + x rs (+- x' rs' of the block's other chunk),
  // one v_fma_mix_f32 per term and column, the sign in the rs halves
  float pz = 0.f;
  __asm__("" : "+v"(pz));
  float b[4] = {pz, pz, pz, pz};
  if (a.hb > kChunkCols && a.hb <= 2 * kChunkCols) {
    // second chunk of the block: row 1 of H_2, the other chunk's term negated
    const uint32_t sgn = (cs & (a.hb - 1)) != 0 ? 0x80008000u : 0u;
    const uint32_t x0 = f.x[k][1][0], x1 = f.x[k][1][1];
    const uint32_t r0 = f.r[k][1][0] ^ sgn, r1 = f.r[k][1][1] ^ sgn;
    b[0] = __builtin_fmaf(hlo(x0), hlo(r0), pz);
    b[1] = __builtin_fmaf(hhi(x0), hhi(r0), pz);
    b[2] = __builtin_fmaf(hlo(x1), hlo(r1), pz);
    b[3] = __builtin_fmaf(hhi(x1), hhi(r1), pz);
  }
  // (p + (0 + b) here, (0 + p) + b before: equal for every sign of zero,
  // and for nonzero terms both are the one rounding of an exact sum)
  const uint32_t x0 = f.x[k][0][0], x1 = f.x[k][0][1], r0 = f.r[k][0][0], r1 = f.r[k][0][1];
  v[0] = __builtin_fmaf(hlo(x0), hlo(r0), b[0]);
  v[1] = __builtin_fmaf(hhi(x0), hhi(r0), b[1]);
  v[2] = __builtin_fmaf(hlo(x1), hlo(r1), b[2]);
  v[3] = __builtin_fmaf(hhi(x1), hhi(r1), b[3]);
}

__device__ __forceinline__ void store4h(uint16_t* p, const float v[4]) {
  u32x2_t w = {(uint32_t)f2h(v[0]) | ((uint32_t)f2h(v[1]) << 16), (uint32_t)f2h(v[2]) | ((uint32_t)f2h(v[3]) << 16)};
  *reinterpret_cast<u32x2_t*>(p) = w;
}

// z of every batch row for blocks of 2^LOGH = 1024..4096 columns (the BIG
// variants, which stage whole rows): each row's 4096-column tiles one after
// the other (the last one partial when d is no multiple of 4096: its
// missing columns are whole blocks, loaded as zeros and not stored), all 16
// waves on a tile, four columns per thread: column 256 w + 4 m(l) + j of
// the tile.  Butterflies at distance 1, 2 in registers, 4 .. 128 across
// lanes (the lane stages of tp_rotate_tile.h), 256 .. 2048 across the
// waves as radix-4 steps through `scr` (w bits 0, 1, then 2, 3) -- every
// butterfly the reference's, in its order, so z is the reference's bit for
// bit (and the same z as the stack rotation's).
template <int LOGH, int NPRE>
__device__ void lin_stage_big(const LinArgs& a, const LinPart& P, const XPre<NPRE>& f, bool pre, uint16_t* zl,
                              float* scr, int wave, int lane) {
  static_assert(LOGH >= 10 && LOGH <= 12, "blocks of 1024 .. 4096 columns");
  const int tpr = (a.d + kRotTile - 1) / kRotTile;  // tiles per batch row
  const int m = rot_lane_index(lane), lane4 = 4 * lane;
  const int colw = 256 * wave + 4 * m;  // this thread's columns inside a tile
  const __amdgpu_buffer_rsrc_t xrs = buffer_rsrc(P.x, (uint32_t)((a.batch - 1) * P.ldx + a.d) * 2u);
  const __amdgpu_buffer_rsrc_t rrs = buffer_rsrc(P.rs, (uint32_t)a.d * 2u);
  const float c = a.hdiv, r = a.hrecip;
  // radix-4 step over wave bits s, s + 1 (column distances 256 << s and
  // 512 << s): u_k = the value of wave (w with those bits = k), then the
  // natural-order H_4 row of this wave's two bits (distance 256 << s first)
  auto radix4 = [&](float* v, int s) __attribute__((always_inline)) {
    __syncthreads();  // earlier reads of scr are done
    *reinterpret_cast<float4_t*>(scr + colw) = float4_t{v[0], v[1], v[2], v[3]};
    __syncthreads();
    const int base = colw - 256 * (wave & (3 << s));
    const float s1 = ((wave >> s) & 1) ? -1.f : 1.f, s2 = ((wave >> (s + 1)) & 1) ? -1.f : 1.f;
    const float4_t u0 = *reinterpret_cast<const float4_t*>(scr + base);
    const float4_t u1 = *reinterpret_cast<const float4_t*>(scr + base + (256 << s));
    const float4_t u2 = *reinterpret_cast<const float4_t*>(scr + base + (512 << s));
    const float4_t u3 = *reinterpret_cast<const float4_t*>(scr + base + (768 << s));
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float s01 = __builtin_fmaf(s1, u1[e], u0[e]);
      const float s23 = __builtin_fmaf(s1, u3[e], u2[e]);
      v[e] = __builtin_fmaf(s2, s23, s01);
    }
  };
  // One tile: batch row b, tile tcol, this thread's words xw, rw.
  auto tile = [&](int b, int tcol, const u32x2_t xw, const u32x2_t rw) __attribute__((always_inline)) {
    const int col = tcol * kRotTile + colw;
    const bool ok = col < a.d;
    float v[4];
    rot_products<true, 1>(&xw, &rw, v);
    rot_reg_stage<2, 2, LOGH, 4>(v);
    rot_lane_stage<0, LOGH, 4>(v, m, lane4);
    rot_lane_stage<1, LOGH, 4>(v, m, lane4);
    rot_lane_stage<2, LOGH, 4>(v, m, lane4);
    rot_lane_stage<3, LOGH, 4>(v, m, lane4);
    rot_lane_stage<4, LOGH, 4>(v, m, lane4);
    rot_lane_stage<5, LOGH, 4>(v, m, lane4);
    radix4(v, 0);  // distances 256, 512
    if constexpr (LOGH == 11) {  // distance 1024: wave bit 2
      __syncthreads();
      *reinterpret_cast<float4_t*>(scr + colw) = float4_t{v[0], v[1], v[2], v[3]};
      __syncthreads();
      const float s1 = ((wave >> 2) & 1) ? -1.f : 1.f;
      const float4_t p = *reinterpret_cast<const float4_t*>(scr + (colw ^ 1024));
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = __builtin_fmaf(s1, v[e], p[e]);
    } else if constexpr (LOGH == 12) {
      radix4(v, 2);  // distances 1024, 2048
    }
    if (ok) *reinterpret_cast<u32x2_t*>(zl + b * a.zstride + col) = rot_z4<LOGH>(v, c, r);
  };
  // The first tile from the words lin_prefetch_big loaded ahead of the
  // weights (a copy of its own: inside the loop, the wait before the tile's
  // words would also cover every weight load), then the rest.
  int it0 = 0;
  if (pre) {
    tile(0, 0, f.x[0][0], f.r[0][0]);
    it0 = 1;
  }
  for (int it = it0; it < a.batch * tpr; ++it) {
    int tcol = 0;
    const int b = udiv_small(it, tpr, &tcol);  // (it < batch * tpr)
    const int col = tcol * kRotTile + colw;
    const bool ok = col < a.d;
    tile(b, tcol, load4h_words(xrs, ok ? (uint32_t)(b * P.ldx + col) : kOutOfRange / 2u),
         load4h_words(rrs, ok ? (uint32_t)col : kOutOfRange / 2u));
  }
}

// BIG: this thread's words of the first tile (batch row 0, columns
// 256 w + 4 m(l) ..), loaded before the weights so that staging it waits for
// them only.
template <int NPRE>
__device__ __forceinline__ XPre<NPRE> lin_prefetch_big(const LinArgs& a, const LinPart& P, int wave, int lane) {
  XPre<NPRE> f;
  const __amdgpu_buffer_rsrc_t xrs = buffer_rsrc(P.x, (uint32_t)((a.batch - 1) * P.ldx + a.d) * 2u);
  const __amdgpu_buffer_rsrc_t rrs = buffer_rsrc(P.rs, (uint32_t)a.d * 2u);
  const int col = 256 * wave + 4 * rot_lane_index(lane);
  const bool ok = col < a.d;
  f.x[0][0] = load4h_words(xrs, ok ? (uint32_t)col : kOutOfRange / 2u);
  f.r[0][0] = load4h_words(rrs, ok ? (uint32_t)col : kOutOfRange / 2u);
  return f;
}

// Stage z rows [0, batch) x columns [pu0 * 256, (pu0 + npu) * 256) of linear
// P in LDS (column pu0 * 256 at LDS column 0; the BIG variant stages whole
// rows: pu0 = 0, npu = G4).
// Blocks of 1024..4096 columns (d a multiple of 1024, so G4 * 256 == d) go
// through `scr` one batch row at a time: H_256 inside every chunk (fp32),
// then H_(hb/256) across the chunks of each block -- the stages in order of
// distance, as the reference's transform runs them.
// BIG: the kernel variant for blocks above 512 columns (the only one that
// holds that path's registers); the others take blocks <= 512 only.
template <bool ROT, bool BIG, int NPRE>
__device__ void lin_stage_z(const LinArgs& a, const LinPart& P, const XPre<NPRE>& f, bool pre, int pu0, int npu,
                            uint32_t rnpu, uint16_t* zl, float* scr, int tid, int wave, int lane) {
  const int nch = npu;
  if constexpr (!ROT) {
    const int per_row = nch * kChunkCols / 8;
    for (int i = tid; i < a.batch * per_row; i += kLinThreads) {
      const int b = i / per_row, c8 = (i - b * per_row) * 8;
      *reinterpret_cast<u32x4_t*>(zl + b * a.zstride + c8) =
          *(const TP_GLOBAL u32x4_t*)(P.x + (size_t)b * P.ldx + pu0 * kChunkCols + c8);
    }
    return;
  }
  if constexpr (!BIG) {
    int it0 = wave;
    if (pre) {
#pragma unroll
      for (int k = 0; k < NPRE; ++k) {
        const int it = wave + kLinWaves * k;
        if (it < a.batch * nch) {
          const int b = udiv_recip(it, rnpu);  // (it < batch * nch)
          const int ci = it - b * nch;
          float v[4];
          lin_pre_product(a, f, k, (pu0 + ci) * kChunkCols, v);
          lin_chunk_fwht(a, lane, v);
          store4h(zl + b * a.zstride + ci * kChunkCols + lane * 4, v);
        }
      }
      it0 = wave + kLinWaves * NPRE;
    }
    for (int it = it0; it < a.batch * nch; it += kLinWaves) {
      const int b = udiv_recip(it, rnpu);  // (it < batch * nch)
      const int ci = it - b * nch;
      float v[4];
      lin_rotate_chunk(a, P, b, (pu0 + ci) * kChunkCols, lane, v);
      store4h(zl + b * a.zstride + ci * kChunkCols + lane * 4, v);
    }
    return;
  } else {
    const int logh = __builtin_ctz((unsigned)a.hb);  // 10, 11 or 12 (uniform)
    if (logh == 10) lin_stage_big<10>(a, P, f, pre, zl, scr, wave, lane);
    else if (logh == 11) lin_stage_big<11>(a, P, f, pre, zl, scr, wave, lane);
    else lin_stage_big<12>(a, P, f, pre, zl, scr, wave, lane);
  }
}

// MULTI: 2..4 linears (part of a group is found per tile group); otherwise
// one linear, whose argument fields sit at fixed offsets and load at once.
// BIG: Hadamard blocks of 1024..4096 columns (lin_stage_z).
// KSPLIT: one linear, K cut into a.kparts parts (work item = tile group x
// part); not with MULTI or BIG.
template <int KB, int NS, int SB, bool ROT, bool MULTI, bool BIG, bool KSPLIT>
__global__ void __launch_bounds__(kLinThreads) tcq_linear_kernel(const LinArgs a) {
  static_assert(!(KSPLIT && (MULTI || BIG)), "K-split runs one linear with blocks <= 512");
  __shared__ __attribute__((aligned(16))) uint32_t table[kTableWords];
  extern __shared__ __attribute__((aligned(16))) char lin_lds[];
  constexpr int MW = member_words(KB);
  constexpr int SLOTS = 16 / SB;
  constexpr int NZ = 8 / SLOTS;
  constexpr uint32_t unit_p = 4u * kTileRows * 8u;       // path bytes per unit of a tile
  constexpr uint32_t unit_m = 4u * kTileRows * MW * 4u;  // member bytes per unit of a tile
  // Every kernel argument the prologue uses, in one round trip to the
  // argument segment (one asm statement naming them, before any use; the
  // memory clobber keeps the loads below it).  Left to the compiler, the
  // codebook entry's load went first and its address wait held back the
  // other argument loads, and a multi-linear launch chained one round trip
  // per part: each ~1-2 us before the first weight load.  Not in the BIG
  // variants: there the forced loads spilled scalar registers and the
  // launch got slower (c1 q_proj 8.4 -> 8.7 us).
  const uint16_t* const codebook = a.codebook;
  if constexpr (BIG) {
  } else if constexpr (MULTI) {
    __asm__ volatile("" ::"s"(codebook), "s"(a.d), "s"(a.hb), "s"(a.batch), "s"(a.tpw), "s"(a.zstride),
                     "s"(a.hdiv), "s"(a.G4), "s"(a.c), "s"(a.s), "s"(a.g0[1]), "s"(a.g0[2]),
                     "s"(a.g0[3]), "s"(a.r_s), "s"(a.r_pu_last)
                     : "memory");
  } else if constexpr (KSPLIT) {
    const LinPart& P0 = a.part[0];
    __asm__ volatile("" ::"s"(codebook), "s"(a.d), "s"(a.hb), "s"(a.batch), "s"(a.tpw), "s"(a.zstride),
                     "s"(a.hdiv), "s"(a.G4), "s"(a.c), "s"(a.s), "s"(a.kparts), "s"(a.pu), "s"(a.groups),
                     "s"(a.r_s), "s"(a.r_kparts), "s"(a.r_pu), "s"(a.r_pu_last), "s"(P0.path), "s"(P0.member),
                     "s"(P0.x), "s"(P0.rs), "s"(P0.scales), "s"(P0.n), "s"(P0.T), "s"(P0.ldx), "s"(a.kws),
                     "s"(a.kcnt)
                     : "memory");
  } else {
    const LinPart& P0 = a.part[0];
    __asm__ volatile("" ::"s"(codebook), "s"(a.d), "s"(a.hb), "s"(a.batch), "s"(a.tpw), "s"(a.zstride),
                     "s"(a.hdiv), "s"(a.G4), "s"(a.c), "s"(a.s), "s"(a.r_s), "s"(a.r_pu_last), "s"(P0.path),
                     "s"(P0.member), "s"(P0.x),
                     "s"(P0.rs), "s"(P0.scales), "s"(P0.n), "s"(P0.T), "s"(P0.g0)
                     : "memory");
  }
  uint16_t* zl = reinterpret_cast<uint16_t*>(lin_lds);
  float* scr = reinterpret_cast<float*>(lin_lds + (((size_t)a.batch * a.zstride * 2 + 15) & ~(size_t)15));

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, q = lane >> 4;
  const int slot = r / SB, bb = r % SB;
  const uint32_t laneoff = lane_offsets<KB>(lane);
  const uint32_t pv = (uint32_t)(q * kTileRows + r) * 8u;
  const uint32_t mv = (uint32_t)(q * kTileRows + r) * MW * 4u;
  // B operand halves of this lane inside a unit's staged z (rows past the
  // batch read row 0: their MFMA columns are never written out).
  const int bbz = bb < a.batch ? bb : 0;
  const int zrow = bbz * a.zstride + q * kSegCols;
  // (wave-uniform values are pinned to scalar registers: left to the
  // compiler, the tile index reached the buffer descriptors as a vector
  // value, and every weight load went into a waterfall loop)
  const int lt = __builtin_amdgcn_readfirstlane(udiv_recip(wave, a.r_s));  // local tile of this wave
  const int j = __builtin_amdgcn_readfirstlane(wave - lt * a.s);            // K chunk of this wave (inside the K part)
  const uint32_t tile_p = (uint32_t)a.G4 * unit_p;  // path bytes of one tile
  const uint32_t tile_m = (uint32_t)a.G4 * unit_m;  // member bytes of one tile
  int staged = -1;

  // One tile group.  The first call (the workgroup's own group; the host
  // gives every workgroup one group when they fit) is a copy of its own, so
  // that its loads are scheduled from the kernel's entry state rather than
  // from the merged state of a loop: at the loop head the wait before the
  // weight loads also covered the activation prefetch.
  auto group = [&](const int w) __attribute__((always_inline)) {
    // Work item w: tile group g, K part kp of units [pu0, pu0 + npu).
    int g = w, kp = 0;
    if constexpr (KSPLIT) {
      g = udiv_recip(w, a.r_kparts);
      kp = w - g * a.kparts;
    }
    const int pu0 = KSPLIT ? kp * a.pu : 0;
    const int npu = KSPLIT ? min(a.pu, a.G4 - pu0) : a.G4;
    const uint32_t rnpu = (KSPLIT && kp + 1 < a.kparts) ? a.r_pu : a.r_pu_last;
    const int u0 = __builtin_amdgcn_readfirstlane(pu0 + j * a.c);
    const int nu = __builtin_amdgcn_readfirstlane(min(a.c, pu0 + npu - u0));
    // The group's linear: the parts' first groups ascend and unused parts
    // start at `groups`, so it is the number of parts 1.. starting at or
    // before g.  (Computed from values of one argument round trip, then one
    // indexed load of that part: a select per part made a dependent round
    // trip each.)
    int p = 0;
    if constexpr (MULTI) {
#pragma unroll
      for (int i = 1; i < kLinMaxParts; ++i) p += g >= a.g0[i] ? 1 : 0;
      p = __builtin_amdgcn_readfirstlane(p);
    }
    const LinPart P = a.part[p];
    const int t = __builtin_amdgcn_readfirstlane((g - P.g0) * a.tpw + lt);
    const bool active = lt < a.tpw && t < P.T && nu > 0;  // wave-uniform
    const int tt = __builtin_amdgcn_readfirstlane(active ? t : 0);
    const int key = p + kLinMaxParts * kp;  // what the LDS z holds
    // The first group's activations load before its weights (they gate the
    // rotation, which every decode waits for).
    const bool pre = ROT && key != staged && w == (int)blockIdx.x;
    XPre<lin_pre(KB)> xf;
    if constexpr (ROT && !BIG) {
      if (pre) xf = lin_prefetch_x<lin_pre(KB)>(a, P, pu0, npu, rnpu, wave, lane);
    } else if constexpr (ROT && BIG) {
      if (pre) xf = lin_prefetch_big<lin_pre(KB)>(a, P, wave, lane);
    }

    // Every weight load of this wave, then the halo word (path word 1 of
    // the unit before the chunk, K block 3 lanes) and the row scales.
    const __amdgpu_buffer_rsrc_t prs =
        buffer_rsrc(reinterpret_cast<const char*>(P.path) + (size_t)(uint32_t)tt * tile_p, tile_p);
    const __amdgpu_buffer_rsrc_t mrs =
        buffer_rsrc(reinterpret_cast<const char*>(P.member) + (size_t)(uint32_t)tt * tile_m, tile_m);
    constexpr int MAXU = lin_max_units(MULTI);
    UnitRegs<MW, NZ> R[MAXU];
    const uint32_t su0 = (uint32_t)u0;
    const int lim = active ? nu : 0;  // units of this wave that load (wave-uniform)
    // (every unit is loaded, past lim out of range: the vector offset
    // carries the out-of-range bit, so the scalar offset needs no select --
    // the range check fails whatever that offset, which stays below 2^31.
    // Unconditional, so that the number of loads issued after the
    // activation prefetch is the same on every path and the staging's wait
    // for the prefetch does not also wait for these)
#pragma unroll
    for (int u = 0; u < MAXU; ++u) {
      // out-of-range bit unless u < lim: the sign of lim - u - 1 (|lim| <= 4)
      const uint32_t oob = (uint32_t)(lim - u - 1) & kOutOfRange;
      R[u].X = __builtin_amdgcn_raw_buffer_load_b64(prs, pv | oob, (su0 + u) * unit_p, weight_policy(MW));
      R[u].M = MemberBuf<MW>::load(mrs, mv | oob, (su0 + u) * unit_m);
    }
    const uint32_t x1_prev = __builtin_amdgcn_raw_buffer_load_b32(
        prs, (active && u0 > 0) ? pv + 4u : kOutOfRange, (uint32_t)(u0 > 0 ? u0 - 1 : 0) * unit_p, 0);
    const __amdgpu_buffer_rsrc_t srs = buffer_rsrc(P.scales, (uint32_t)P.n * 2u);
    // rows 4q..4q+3 (zero past n; for odd n also row n - 1, which shares its
    // dword with row n: loaded again on its own, and taken for that row)
    const u32x2_t sc = __builtin_amdgcn_raw_buffer_load_b64(srs, (uint32_t)(tt * kTileRows + 4 * q) * 2u, 0, 0);
    const uint16_t sc_last = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(srs, (uint32_t)(P.n - 1) * 2u, 0, 0);

    // (the codebook is read here, after the weight loads: read at entry, the
    // wait for it came before the part's descriptor loads, one more round
    // trip ahead of every weight load)
    if (w == (int)blockIdx.x) build_pair_table_lanes<KB>(table, codebook_lane_scalar<KB>(codebook, lane), tid, kLinThreads);
    if (key != staged) {
      if (staged >= 0) __syncthreads();  // the previous group's reads of z and scr are done
      lin_stage_z<ROT, BIG, lin_pre(KB)>(a, P, xf, pre, pu0, npu, rnpu, zl, scr, tid, wave, lane);
      staged = key;
    }
    __syncthreads();

    if (active) {
      float4_t acc[SLOTS];
#pragma unroll
      for (int s = 0; s < SLOTS; ++s) acc[s] = float4_t{0.f, 0.f, 0.f, 0.f};
      uint32_t prev = x1_prev;
#pragma unroll
      for (int u = 0; u < MAXU; ++u) {
        if (u < nu) {
          const int cbase = (u0 + u - pu0) * kChunkCols;
#pragma unroll
          for (int l = 0; l < NZ; ++l)
            R[u].Z[l] = *reinterpret_cast<const u32x4_t*>(zl + zrow + mfma_col(l * SLOTS + slot) + cbase);
          const uint32_t provide = (q == 3) ? prev : R[u].X[1];
          slot_unit<KB, NS, SB, MW, NZ>(R[u], provide, lane, laneoff, table, acc);
          prev = R[u].X[1];
        }
      }
      // accumulator `slot` holds this lane's column; the slot-0 lanes' sums
      // over the slots of each batch row (the other lanes' values are unused)
      const float4_t v = slot_column_sums<SLOTS, SB>(acc);
      *reinterpret_cast<float4_t*>(scr + (wave * 64 + lane) * 4) = v;
    }
    __syncthreads();
    if (active && j == 0) {
      float4_t v = *reinterpret_cast<const float4_t*>(scr + (wave * 64 + lane) * 4);
      // (chunks of this part that hold units: a short last part has fewer)
      const int sk = KSPLIT ? (kp + 1 < a.kparts ? a.sk : a.sk_last) : a.s;
      for (int k = 1; k < sk; ++k) {
        const float4_t o = *reinterpret_cast<const float4_t*>(scr + ((wave + k) * 64 + lane) * 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] += o[i];
      }
      bool finish = true;
      if constexpr (KSPLIT) {
        if (a.kparts > 1) {
          // This part's sums into its slice with coherent (L2-bypassing)
          // stores, then the tile's counter.  Lanes of slot 0 hold the
          // valid columns: rows 4q..4q+3 of batch column bb.
          float* own = a.kws + ((size_t)kp * P.T + t) * kLinSliceFloats;
          if (slot == 0 && bb < a.batch) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              __hip_atomic_store(own + (4 * q + i) * 8 + bb, v[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
          __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
          uint32_t old = 0;
          if (lane == 0) old = __hip_atomic_fetch_add(a.kcnt + t, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          old = (uint32_t)__builtin_amdgcn_readfirstlane((int)old);
          if (old + 1u == (uint32_t)a.kparts) {  // (wave-uniform) the last part of this tile
            // Every lane owns entries (row, column) = (e / batch, e % batch),
            // e = lane and lane + 64: all parts' values are loaded (coherent
            // loads, all in flight at once) and added in part order, then
            // the slices and the counter are left zero for the next call.
            const int ne = kTileRows * a.batch;
            const __amdgpu_buffer_rsrc_t srs = buffer_rsrc(P.scales, (uint32_t)P.n * 2u);
            // (buffer accesses over the kparts slices: a part past kparts is
            // out of range, reads 0 and drops its store, with no branch;
            // cache policy sc1, as the coherent stores and loads above)
            const __amdgpu_buffer_rsrc_t krs =
                buffer_rsrc(a.kws, (uint32_t)(a.kparts * P.T * kLinSliceFloats) * 4u);
            const uint32_t pstride = (uint32_t)P.T * kLinSliceFloats * 4u;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const int e = lane + 64 * h;
              if (e < ne) {
                const int row = a.r_batch ? (int)__umulhi((uint32_t)e, a.r_batch) : e;  // e / batch
                const int col = e - row * a.batch;
                const int grow = t * kTileRows + row;
                const uint32_t off = ((uint32_t)t * kLinSliceFloats + (uint32_t)(row * 8 + col)) * 4u;
                const uint16_t sv = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(
                    srs, grow < P.n ? (uint32_t)grow * 2u : kOutOfRange, 0, 0);
                float part[kLinMaxKParts];
#pragma unroll
                for (int pp = 0; pp < kLinMaxKParts; ++pp)
                  part[pp] = __builtin_bit_cast(
                      float, __builtin_amdgcn_raw_buffer_load_b32(krs, off + (uint32_t)pp * pstride, 0, kCoherent));
                float sum = part[0];
#pragma unroll
                for (int pp = 1; pp < kLinMaxKParts; ++pp)
                  if (pp < a.kparts) sum += part[pp];
                __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
                for (int pp = 0; pp < kLinMaxKParts; ++pp)
                  __builtin_amdgcn_raw_buffer_store_b32(0u, krs, off + (uint32_t)pp * pstride, 0, kCoherent);
                if (grow < P.n) {
                  uint16_t out = f2h(sum * h2f(sv));
                  if (P.bias) out = f2h(h2f(out) + h2f(gld(P.bias + grow)));
                  gst(P.y + (size_t)col * P.ldy + grow, out);
                }
              }
            }
            if (lane == 0) __hip_atomic_store(a.kcnt + t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
          finish = false;  // (y written above, by the last part only)
        }
      }
      if (finish && slot == 0 && bb < a.batch) {
        const int row0 = t * kTileRows + 4 * q;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = row0 + i;
          if (row >= P.n) continue;
          const uint16_t sv = row == P.n - 1 ? sc_last : (uint16_t)(sc[i >> 1] >> (16 * (i & 1)));
          uint16_t out = f2h(v[i] * h2f(sv));
          if (P.bias) out = f2h(h2f(out) + h2f(gld(P.bias + row)));
          gst(P.y + (size_t)bb * P.ldy + row, out);
        }
      }
    }
  };
  const int items = KSPLIT ? a.groups * a.kparts : a.groups;
  group((int)blockIdx.x);
  for (int w = (int)(blockIdx.x + gridDim.x); w < items; w += (int)gridDim.x) group(w);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
namespace {

template <int KB, int NS, int SB, bool ROT>
void launch_linear(const LinArgs& a, int grid, size_t dyn, hipStream_t s) {
  // (blocks above 512 columns run their own variant, so that the others
  // keep that path's registers free: no spill frame, no scratch set-up; the
  // K-split variant is a third one)
  const bool big = ROT && a.hb > 2 * kChunkCols;
  auto kern = big ? (a.n_part > 1 ? tcq_linear_kernel<KB, NS, SB, ROT, true, ROT, false>
                                  : tcq_linear_kernel<KB, NS, SB, ROT, false, ROT, false>)
                  : (a.n_part > 1 ? tcq_linear_kernel<KB, NS, SB, ROT, true, false, false>
                     : a.kparts > 1 ? tcq_linear_kernel<KB, NS, SB, ROT, false, false, true>
                                    : tcq_linear_kernel<KB, NS, SB, ROT, false, false, false>);
  allow_dynamic_lds(reinterpret_cast<const void*>(kern), kTableBytes + 256);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kLinThreads), dyn, s, a);
}

template <int KB, int NS>
void launch_linear_sb(const LinArgs& a, int grid, size_t dyn, bool rot, hipStream_t s) {
  if (a.batch <= 4)
    rot ? launch_linear<KB, NS, 4, true>(a, grid, dyn, s) : launch_linear<KB, NS, 4, false>(a, grid, dyn, s);
  else
    rot ? launch_linear<KB, NS, 8, true>(a, grid, dyn, s) : launch_linear<KB, NS, 8, false>(a, grid, dyn, s);
}

// One way to cut a linear's work over the chip: K in kparts parts of pu
// units, each part's K range in chunks of c units (sc chunks per tile), tpw
// tiles per group of 16 waves.
struct LinPlan {
  int64_t kparts, pu, c, sc, tpw, groups, items;
  double cost;
};

}  // namespace

int64_t linear_ksplit_bytes(int64_t T) {
  const int64_t tp = std::min<int64_t>(T * kLinMaxKParts, kLinMaxTileParts);
  return tp * kLinSliceFloats * 4 + T * 4;
}

// The cut of the one-pass kernel for n_lin linears of T[i] row tiles over
// G4 units of K (Hadamard block hb when rot), or kparts == 0 when it
// declines the shapes (the split-K kernel runs).  Host only, no device
// state: cus and max_lds describe the device.
LinPlan plan_linear(int n_lin, const int64_t* T, int64_t G4, int64_t d, int64_t hb, bool rot, int64_t batch,
                    int bits, bool can_split, int64_t workspace_bytes, int cus, int64_t max_lds) {
  const bool rows8 = batch > 4;
  const bool big = rot && hb > 2 * kChunkCols;
  const int64_t lds_room = max_lds - kTableBytes - 16;
  // Candidate cuts, priced in us of a latency-bound launch: 1 per unit
  // decoded per wave, 1.3 per staging item per wave among the first
  // lin_pre(bits) (their activations load before the weights), 1.85 per
  // later item (an activation round trip and a rotation chain), and for a
  // K split 2.3 + 0.3 per part (the pass through memory: coherent stores,
  // the tile's counter, the last part's loads), times the rounds when the
  // groups outnumber the CUs.  (Fitted to 21 forced cuts of Qwen3-4B
  // gate_proj and down_proj, k=3, batch 1 / 4 / 8, on one box -- e.g.
  // down_proj batch 4: one part 17.1 us, 3 / 5 / 7 / 10 parts 14.1 / 12.0
  // / 11.9 / 12.5 us; gate_proj batch 1: one part 8.3 us, 2 / 3 parts 9.6 /
  // 10.1 us -- with the split's fixed cost raised from the fit's 1.55 to
  // 2.3 so that gate_proj at batch 4 keeps one part: 10.3 us, 3 parts
  // 10.6 us.)
  //
  // Single part (the whole K range per workgroup): staging issues the
  // activations of lin_pre(bits) items per wave ahead of the weights.
  // Blocks <= 512 columns take up to 6 items per wave before the split-K
  // kernel is the faster one (Qwen3-4B down_proj, k=3, batch 2: 4.75 items,
  // 17.3 -> 14.3 us); larger blocks stage one batch row at a time through
  // LDS: up to 3 items per wave, batch <= 4 (o_proj, 4096-column blocks,
  // batch 4 at 4 items: 18.0 -> 19.6 us).  At batch 5..8 a single part
  // pays off when each workgroup covers several row tiles (gate_proj k=3:
  // 14.2 -> 11.8 us at batch 5, 15.6 -> 14.8 us at batch 8), not with one
  // tile per workgroup (k_proj at batch 8: 10.3 -> 13.3 us).
  //
  // K parts (one linear, blocks <= 512, a workspace for the slices): each
  // part covers whole Hadamard blocks, so a workgroup rotates its own part
  // of the input; every (tile group, part) gets a CU of its own.
  LinPlan best{0, 0, 0, 0, 0, 0, 0, 1e30};
  const int64_t align = (rot && hb > kChunkCols) ? hb / kChunkCols : 1;  // units per Hadamard block
  can_split = can_split && n_lin == 1 && !big;
  int64_t last_kparts = 0;
  const int64_t maxu = lin_max_units(n_lin > 1);
  for (int64_t want = 1; want <= kLinMaxKParts && want <= G4; ++want) {
    int64_t pu = (G4 + want - 1) / want;
    pu = (pu + align - 1) / align * align;
    const int64_t kparts = (G4 + pu - 1) / pu;
    if (kparts == last_kparts) continue;
    last_kparts = kparts;
    if (kparts > 1) {
      if (!can_split || kparts * T[0] > kLinMaxTileParts) continue;
      if (workspace_bytes < kparts * T[0] * kLinSliceFloats * 4 + T[0] * 4) continue;
    }
    // LDS: 64 KiB table (static) + z rows of the part + max(partial sums,
    // one fp32 row); one launch stages every batch row (no weight re-reads)
    const int64_t scr_bytes = std::max<int64_t>(kLinRedBytes, big ? d * 4 : 0);
    if (lds_room - scr_bytes < batch * (pu * kChunkCols + 8) * 2) continue;
    const int64_t items = (batch * pu + kLinWaves - 1) / kLinWaves;  // staging items per wave (blocks <= 512)
    if (kparts == 1) {
      if (pu > (int64_t)kLinWaves * maxu) continue;
      if (batch * pu > (int64_t)kLinWaves * (big ? kLinPre + 1 : 6)) continue;
      if (rows8 && big) continue;
    } else if (items > 6) {
      continue;
    }
    for (int64_t c = (pu + kLinWaves - 1) / kLinWaves; c <= maxu; ++c) {
      const int64_t sc = (pu + c - 1) / c;
      const int64_t tpw = kLinWaves / sc;
      int64_t groups = 0;
      for (int i = 0; i < n_lin; ++i) groups += (T[i] + tpw - 1) / tpw;
      const int64_t wgs = groups * kparts;
      if (wgs > cus && c < maxu) continue;  // one round if a larger c allows it
      if (kparts == 1 && rows8 && tpw < 2) break;
      if (groups > INT32_MAX / (2 * kLinMaxKParts)) break;
      const int64_t pre = std::min<int64_t>(std::max<int64_t>(items, 1), lin_pre(bits));
      const double stage = 1.3 * (double)pre + 1.85 * (double)std::max<int64_t>(items - pre, 0);
      const double rounds = (double)((wgs + cus - 1) / cus);
      const double split = kparts > 1 ? 2.3 + 0.3 * (double)kparts : 0.0;
      const double cost = ((double)c + stage + split) * rounds;
      if (cost < best.cost - 1e-9) best = LinPlan{kparts, pu, c, sc, tpw, groups, items, cost};
      break;  // the smallest c that fits is the cheapest for this cut
    }
  }
  return best;
}

int linear_forward_fast(const TiledLinearArgs* ls, int n_lin, int64_t batch, const uint16_t* codebook,
                        int bits, int n_states, hipStream_t s, bool clear_ws) {
  if (batch < 1 || batch > 8 || n_lin < 1 || n_lin > kLinMaxParts) return kLinearNotHandled;
  if (bits < 2 || bits > 4) return kLinearNotHandled;
  if ((uintptr_t)codebook & 3) return kLinearNotHandled;  // (read as dwords through the scalar cache)
  const bool rot = ls[0].rot_scale != nullptr;
  const int64_t d = ls[0].d, hb = rot ? ls[0].block : 1;
  for (int i = 1; i < n_lin; ++i)
    if (ls[i].d != d || (rot && ls[i].block != hb) || ls[i].x != ls[0].x || ls[i].ldx != ls[0].ldx)
      return kLinearNotHandled;
  if (rot && hb > 4096) return kLinearNotHandled;
  Geom g0;
  if (tiled_geom(ls[0].n, d, bits, &g0) != TP_OK) return kLinearNotHandled;
  const int64_t G4 = g0.G4;
  if (rot && hb > 2 * kChunkCols && G4 * kChunkCols != d) return kLinearNotHandled;
  const bool big = rot && hb > 2 * kChunkCols;
  int64_t T[kLinMaxParts];
  for (int i = 0; i < n_lin; ++i) {
    Geom g;
    if (tiled_geom(ls[i].n, d, bits, &g) != TP_OK) return kLinearNotHandled;
    T[i] = g.T;
  }
  const int cus = device_cu_count();
  const bool ws_ok = ls[0].workspace && !((uintptr_t)ls[0].workspace & 15);
  const LinPlan best = plan_linear(n_lin, T, G4, d, hb, rot, batch, bits, ws_ok,
                                   ws_ok ? ls[0].workspace_bytes : 0, cus, (int64_t)device_max_lds());
  if (best.kparts == 0) return kLinearNotHandled;
  // (the kernel's divisions by reciprocal need x * d < 2^32: work items x
  // K parts; its unit offsets stay below 2^31 up to the last unit loaded)
  if (best.groups * best.kparts * best.kparts >= ((int64_t)1 << 32) ||
      (G4 + kLinMaxUnitsMulti) * (4 * kTileRows * member_words(bits) * 4) >= ((int64_t)1 << 31))
    return kLinearNotHandled;

  const int64_t zstride = best.pu * kChunkCols + 8;
  const int64_t scr = std::max<int64_t>(kLinRedBytes, big ? d * 4 : 0);

  LinArgs a;
  a.codebook = codebook;
  a.n_part = n_lin;
  a.groups = (int32_t)best.groups;
  a.d = (int32_t)d;
  a.G4 = (int32_t)G4;
  a.hb = (int32_t)hb;
  a.c = (int32_t)best.c;
  a.s = (int32_t)best.sc;
  a.tpw = (int32_t)best.tpw;
  a.zstride = (int32_t)zstride;
  a.hdiv = (float)__builtin_sqrt((double)hb);
  a.hrecip = 1.f / a.hdiv;
  a.kparts = (int32_t)best.kparts;
  a.pu = (int32_t)best.pu;
  a.r_s = lin_recip(best.sc);
  a.r_kparts = lin_recip(best.kparts);
  a.r_pu = lin_recip(best.pu);
  a.r_pu_last = lin_recip(G4 - (best.kparts - 1) * best.pu);
  a.sk = (int32_t)((best.pu + best.c - 1) / best.c);
  a.sk_last = (int32_t)((G4 - (best.kparts - 1) * best.pu + best.c - 1) / best.c);
  a.kws = nullptr;
  a.kcnt = nullptr;
  int64_t g0acc = 0;
  for (int i = 0; i < kLinMaxParts; ++i) {
    const TiledLinearArgs& l = ls[i < n_lin ? i : 0];
    LinPart& P = a.part[i];
    P.path = reinterpret_cast<const uint32_t*>(l.path_tiled);
    P.member = reinterpret_cast<const uint32_t*>(l.member_tiled);
    P.rs = rot ? l.rot_scale : nullptr;
    P.scales = l.scales;
    P.bias = l.bias;
    P.n = (int32_t)l.n;
    P.T = (int32_t)T[i < n_lin ? i : 0];
    P.ldx = (int32_t)l.ldx;
    P.ldy = (int32_t)l.ldy;
    P.g0 = (int32_t)(i < n_lin ? g0acc : best.groups);
    P.reserved = 0;
    a.g0[i] = P.g0;
    if (i < n_lin) g0acc += (T[i] + best.tpw - 1) / best.tpw;
  }
  if (best.kparts > 1) {
    const int64_t slices = best.kparts * T[0] * kLinSliceFloats * 4;
    a.kws = reinterpret_cast<float*>(ls[0].workspace);
    a.kcnt = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(ls[0].workspace) + slices);
    if (clear_ws) {
      const int st = zero_device_bytes(ls[0].workspace, slices + T[0] * 4, s);
      if (st) return st;
    }
  }
  const int64_t work = best.groups * best.kparts;
  const int grid = (int)std::min<int64_t>(work, cus);
  a.batch = (int32_t)batch;
  a.r_batch = lin_recip(batch);
  for (int i = 0; i < kLinMaxParts; ++i) {
    const TiledLinearArgs& l = ls[i < n_lin ? i : 0];
    a.part[i].x = l.x;
    a.part[i].y = l.y;
  }
  const size_t dyn = (size_t)((batch * zstride * 2 + 15) & ~(int64_t)15) + (size_t)scr;
  switch (bits * 100 + n_states) {
    case 204: launch_linear_sb<2, 4>(a, grid, dyn, rot, s); break;
    case 208: launch_linear_sb<2, 8>(a, grid, dyn, rot, s); break;
    case 216: launch_linear_sb<2, 16>(a, grid, dyn, rot, s); break;
    case 264: launch_linear_sb<2, 64>(a, grid, dyn, rot, s); break;
    case 304: launch_linear_sb<3, 4>(a, grid, dyn, rot, s); break;
    case 308: launch_linear_sb<3, 8>(a, grid, dyn, rot, s); break;
    case 316: launch_linear_sb<3, 16>(a, grid, dyn, rot, s); break;
    case 364: launch_linear_sb<3, 64>(a, grid, dyn, rot, s); break;
    case 404: launch_linear_sb<4, 4>(a, grid, dyn, rot, s); break;
    case 408: launch_linear_sb<4, 8>(a, grid, dyn, rot, s); break;
    case 416: launch_linear_sb<4, 16>(a, grid, dyn, rot, s); break;
    case 464: launch_linear_sb<4, 64>(a, grid, dyn, rot, s); break;
    default: return TP_ERR_UNSUPPORTED_STATES;
  }
  return launch_status();
}

}  // namespace tp

using namespace tp;

extern "C" int tp_linear_forward_plan(const int64_t* ns, int n_linears, int64_t d, int64_t block, int bits,
                                      int64_t batch, int64_t workspace_bytes, int cus, int64_t lds_bytes,
                                      int64_t* out) {
  if (!ns || !out) return TP_ERR_NULL_POINTER;
  for (int i = 0; i < 6; ++i) out[i] = 0;
  if (n_linears < 1 || n_linears > kLinMaxParts || cus < 1 || lds_bytes < 1 || d < 1) return TP_ERR_BAD_DIMS;
  if (bits < 2 || bits > 4) return TP_ERR_UNSUPPORTED_BITS;
  if (block < 1 || (block & (block - 1)) || d % block) return TP_ERR_BAD_BLOCK;
  if (batch < 1 || batch > 8 || block > 4096) return TP_OK;  // not the one-pass kernel's
  Geom g0;
  int st = tiled_geom(ns[0], d, bits, &g0);
  if (st) return st;
  if (block > 2 * kChunkCols && g0.G4 * kChunkCols != d) return TP_OK;
  int64_t T[kLinMaxParts];
  for (int i = 0; i < n_linears; ++i) {
    Geom g;
    st = tiled_geom(ns[i], d, bits, &g);
    if (st) return st;
    T[i] = g.T;
  }
  const LinPlan p = plan_linear(n_linears, T, g0.G4, d, block, true, batch, bits, workspace_bytes > 0,
                                workspace_bytes, cus, lds_bytes);
  if (p.kparts == 0) return TP_OK;
  out[0] = p.kparts;
  out[1] = p.pu;
  out[2] = p.c;
  out[3] = p.sc;
  out[4] = p.tpw;
  out[5] = p.groups * p.kparts;
  return TP_OK;
}

