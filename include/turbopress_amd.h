/* turbopress_amd: MI355X (gfx950) kernels for TurboPress's packed-TCQ decode path.
 *
 * C ABI of libturbopress_amd.so.  Every entry point takes plain device
 * pointers, sizes in elements or bytes, and a hipStream_t passed as void*.
 * None allocates memory, none synchronises the host, and none autotunes, so
 * all device entry points may be recorded into a HIP graph.  All return an
 * int status (TP_OK == 0); tp_status_string() names it.
 *
 * Data formats follow the reference's format v2 (turbopress/runtime.py:73-100,
 * 171-186): fp16 values are passed as raw uint16 bit patterns, packed streams
 * are little-endian bit streams with each row padded to whole bytes.
 *
 * Reference paths below are relative to the TurboPress 0.5.2 checkout.
 */
#ifndef TURBOPRESS_AMD_H
#define TURBOPRESS_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TP_ABI_VERSION 1

enum tp_status {
  TP_OK = 0,
  TP_ERR_NULL_POINTER = 1,        /* a required pointer is NULL */
  TP_ERR_UNSUPPORTED_BITS = 2,    /* bits outside what the entry point supports */
  TP_ERR_UNSUPPORTED_STATES = 3,  /* n_states not in {4, 8, 16, 64} */
  TP_ERR_BAD_DIMS = 4,            /* non-positive or inconsistent sizes */
  TP_ERR_MISALIGNED = 5,          /* pointer or stride alignment violated */
  TP_ERR_BAD_BLOCK = 6,           /* Hadamard block not a power of 2 dividing d, or too large */
  TP_ERR_HIP = 7,                 /* a HIP launch or query failed */
  TP_ERR_WORKSPACE = 8,           /* workspace missing or too small */
  TP_ERR_BAD_LAYOUT = 9           /* device-layout descriptor inconsistent with the call */
};

/* ABI version of the loaded library (TP_ABI_VERSION when headers match). */
int tp_abi_version(void);

/* Static, human-readable name of a status code. */
const char* tp_status_string(int status);

/* Read `bytes` (a multiple of 16, 16-byte aligned) of device memory once
 * with a plain streaming-read kernel (each wave streams a contiguous slice
 * with 16-byte loads, 2 workgroups of 8 waves per CU); `sink` (one device
 * word) is written only in the practically impossible case that the XOR of
 * all words hits a constant.
 * Benchmark utility: the achievable read bandwidth of the GPU it runs on,
 * the practical ceiling of an HBM-bound read stream.  No reference
 * counterpart. */
int tp_read_probe(const void* buf, int64_t bytes, uint32_t* sink, void* stream);

/* ---------------------------------------------------------------------------
 * Trellis tables (host only, no GPU work)
 * ------------------------------------------------------------------------- */

/* Window -> subset LUT of the S-state trellis, lut_len >= 2*S entries.
 * Replaces turbopress/runtime.py:106-119 (subset_lut) over
 * turbopress/trellis.py:64-80 (Trellis.subset_table). */
int tp_subset_lut(int n_states, uint8_t* lut_out, int lut_len);

/* ---------------------------------------------------------------------------
 * Rotation
 * ------------------------------------------------------------------------- */

/* z = blockFWHT(x * rot_scale): orthonormal Sylvester Walsh-Hadamard transform
 * applied independently to each contiguous `block` of the last dimension,
 * computed in fp32 and stored as fp16.  x, z: fp16 [batch, d] row-major
 * (z may not alias x); rot_scale: fp16 [d].  block must be a power of 2
 * dividing d, at most 16384.
 * Replaces turbopress/triton_kernel.py:235-260 (fwht_scale); the math is
 * turbopress/runtime.py:192-208 and turbopress/hadamard.py:37-56. */
int tp_fwht_scale(const uint16_t* x, const uint16_t* rot_scale, uint16_t* z,
                  int64_t batch, int64_t d, int64_t block, void* stream);

/* tp_fwht_scale writing z with row stride ldz >= d and zero-filling columns
 * [d, ldz) -- the zero-padded activation layout tp_tcq_gemv_tiled reads
 * (ldz = the z_cols reported by tp_tiled_layout). */
int tp_fwht_scale_padded(const uint16_t* x, const uint16_t* rot_scale, uint16_t* z,
                         int64_t batch, int64_t d, int64_t block, int64_t ldz, void* stream);

/* out = blockFWHT(x * pre_scale) * post_scale over `rows` rows of length d
 * (either scale may be NULL), fp32 butterflies, fp16 in/out.  With
 * pre_scale = NULL and post_scale = rot_scale this is the load-time fold of
 * decoded rotated weights back to the original basis,
 * turbopress/runtime.py:282-286 (mode "cached"); with post_scale = NULL it is
 * tp_fwht_scale. */
int tp_block_fwht_rows(const uint16_t* x, const uint16_t* pre_scale,
                       const uint16_t* post_scale, uint16_t* out,
                       int64_t rows, int64_t d, int64_t block, void* stream);

/* ---------------------------------------------------------------------------
 * Decode (natural format v2 streams)
 * ------------------------------------------------------------------------- */

/* levels[r, c] = member[r, c] * 4 + LUT[window(r, c)] for n_rows rows, as
 * uint8 [n_rows, out_stride].  path: [n_rows, path_stride] bytes (1 bit per
 * weight); member: [n_rows, member_stride] bytes ((bits-1) bits per weight),
 * or NULL when bits == 1.  bits in [1, 7].
 * Replaces turbopress/runtime.py:122-139 (window_decode_levels) applied to
 * turbopress/runtime.py:93-100 (unpack_le) of the packed streams. */
int tp_window_decode_levels(const uint8_t* path, int64_t path_stride,
                            const uint8_t* member, int64_t member_stride,
                            int64_t n_rows, int64_t d, int bits, int n_states,
                            uint8_t* levels_out, int64_t out_stride, void* stream);

/* w[r, c] = fp16(f32(codebook[level[r, c]]) * f32(scales[r])), the rotated
 * weight rows of a packed linear, fp16 [n_rows, out_stride].  The pointers
 * address the first row to decode (a row slice is a pointer offset).
 * Replaces turbopress/runtime.py:291-301 (PackedTCQLinear.decode_rows). */
int tp_decode_rows(const uint8_t* path, int64_t path_stride,
                   const uint8_t* member, int64_t member_stride,
                   const uint16_t* scales, const uint16_t* codebook,
                   int64_t n_rows, int64_t d, int bits, int n_states,
                   uint16_t* w_out, int64_t out_stride, void* stream);

/* ---------------------------------------------------------------------------
 * GEMV on natural format v2 streams (any bits in [1, 7], any S, any batch)
 * ------------------------------------------------------------------------- */

/* y[b, r] = fp16(scale[r] * sum_c codebook[level[r, c]] * z[b, c]) (+ bias[r]
 * added in fp16 as the reference does), fp32 accumulation.  z: fp16 [batch, d]
 * rotated activations; y: fp16 [batch, n]; bias may be NULL.
 * Replaces turbopress/triton_kernel.py:132-157 (packed_gemv) followed by
 * turbopress/runtime.py:332-333 (bias). */
int tp_tcq_gemv(const uint16_t* z, int64_t batch,
                const uint8_t* path, int64_t path_stride,
                const uint8_t* member, int64_t member_stride,
                const uint16_t* scales, const uint16_t* codebook, const uint16_t* bias,
                int64_t n, int64_t d, int bits, int n_states,
                uint16_t* y, void* stream);

/* ---------------------------------------------------------------------------
 * Bandwidth path: device layout + MFMA decode-GEMV (bits 2, 3 and 4)
 * ------------------------------------------------------------------------- */

/* Geometry of the device layout of an n x d linear at `bits`: 16-row tiles,
 * 64-column segments (padded to a multiple of 4).  Reports the tile and
 * segment counts, the byte sizes of the re-tiled path and member streams
 * (exactly n_pad * d_pad * bits / 8 together), and the padded activation
 * width z_cols.  Any output pointer may be NULL.  Host only.
 * Replaces the load-time stream build of turbopress/runtime.py:253-277
 * (mode "triton"), which re-packed (k+1)-bit level codes; this layout stays
 * at the true k bits per weight. */
int tp_tiled_layout(int64_t n, int64_t d, int bits, int64_t* tiles, int64_t* segments,
                    int64_t* path_bytes, int64_t* member_bytes, int64_t* z_cols);

/* Re-tile the natural format-v2 path/member streams of an n x d linear into
 * the device layout (both outputs 16-byte aligned, sizes from
 * tp_tiled_layout).  Bijective on the weights; padding is zero.
 * Replaces turbopress/runtime.py:253-277. */
int tp_retile(const uint8_t* path, int64_t path_stride, const uint8_t* member,
              int64_t member_stride, int64_t n, int64_t d, int bits,
              uint8_t* path_tiled, uint8_t* member_tiled, void* stream);

/* Bytes of workspace tp_tcq_gemv_tiled / tp_packed_linear_forward may use
 * for n rows at `batch` (0 for invalid sizes: n outside [1, 2^30], batch
 * outside [1, 32]): the fp32 split-K sums of the batch 5..32 kernels or the
 * per-part slices of a K-split batch <= 8 launch, and their counters.  The
 * workspace must be zero before the first call; every call leaves it zero
 * again, so one allocation serves any number of calls (and graph replays)
 * on one stream, also of linears of other sizes up to n. */
int64_t tp_gemv_workspace_bytes(int64_t n, int64_t batch);

/* y[b, r] = fp16(scale[r] * sum_c codebook[level[r, c]] * z[b, c]) (+ bias),
 * reading the device layout.  z: fp16 [batch, ldz] rotated activations, zero
 * in columns [d, ldz), ldz >= z_cols and a multiple of 8, 16-byte aligned;
 * y: fp16 [batch, ldy]; batch in [1, 32]; bits in {2, 3, 4}; n_states in
 * {4, 8, 16, 64}.  Calls that overlap on one workspace race.
 * Replaces turbopress/triton_kernel.py:132-157 (packed_gemv). */
int tp_tcq_gemv_tiled(const uint16_t* z, int64_t ldz, int64_t batch,
                      const uint8_t* path_tiled, const uint8_t* member_tiled,
                      const uint16_t* scales, const uint16_t* codebook, const uint16_t* bias,
                      int64_t n, int64_t d, int bits, int n_states,
                      uint16_t* y, int64_t ldy, void* workspace, int64_t workspace_bytes,
                      void* stream);

/* Fused PackedTCQLinear forward on the device layout: rotation of x
 * (z = blockFWHT(x * rot_scale), Hadamard block `block`) computed per
 * workgroup in LDS for the K range it streams, then the decode-GEMV, bias add
 * and fp16 output, in ONE kernel launch.  x: fp16 [batch, ldx] (ldx and d
 * multiples of 4, 8-byte aligned); other arguments as tp_tcq_gemv_tiled.
 * At batch <= 8 a 4-byte aligned codebook takes the one-pass kernel (which
 * reads it as dwords through the scalar cache); any other runs the earlier
 * tiled kernels, with the same results.
 * Replaces turbopress/runtime.py:312-316 + 332-333 (fwht_scale, packed_gemv,
 * bias). */
int tp_packed_linear_forward(const uint16_t* x, int64_t ldx, int64_t batch,
                             const uint16_t* rot_scale, int64_t block,
                             const uint8_t* path_tiled, const uint8_t* member_tiled,
                             const uint16_t* scales, const uint16_t* codebook,
                             const uint16_t* bias, int64_t n, int64_t d, int bits,
                             int n_states, uint16_t* y, int64_t ldy, void* workspace,
                             int64_t workspace_bytes, void* stream);

/* tp_packed_linear_forward without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  No counterpart in the reference.
 * The workspace is a fixed device array inside the library (2 MiB + 8 KiB),
 * one per GPU, held until the process ends: it holds the split-K sums of n
 * up to 16384 rows at any batch <= 32 (32768 at batch <= 16); a call whose
 * route would need more returns TP_ERR_WORKSPACE before any launch (calls
 * whose route needs no workspace, e.g. most batch-1 shapes, have no limit).
 * Each launch that uses the array is preceded by a fill kernel clearing the
 * bytes it uses; the call allocates nothing.  The first call on a device
 * looks the array up (not capturable: make one call per device before
 * capturing).  Calls that overlap on one GPU race. */
int tp_packed_linear_forward_noalloc(const uint16_t* x, int64_t ldx, int64_t batch,
                                     const uint16_t* rot_scale, int64_t block,
                                     const uint8_t* path_tiled, const uint8_t* member_tiled,
                                     const uint16_t* scales, const uint16_t* codebook,
                                     const uint16_t* bias, int64_t n, int64_t d, int bits,
                                     int n_states, uint16_t* y, int64_t ldy, void* stream);

/* Host only: the cut the batch <= 8 one-pass kernel of
 * tp_packed_linear_forward / tp_packed_linear_forward_group takes for
 * n_linears linears of ns[i] rows sharing d columns (Hadamard block
 * `block`), on a device of `cus` compute units and `lds_bytes` of LDS per
 * workgroup, with a workspace of workspace_bytes (0: none).  out[0..5] =
 * K parts (0: the kernel declines; the split-K kernel runs), 256-column
 * units per part, units per wave, chunks per row tile, row tiles per
 * workgroup, workgroups.  No reference counterpart: it reports the
 * library's planning (tests and tuning). */
int tp_linear_forward_plan(const int64_t* ns, int n_linears, int64_t d, int64_t block, int bits,
                           int64_t batch, int64_t workspace_bytes, int cus, int64_t lds_bytes,
                           int64_t* out);

/* One launch for up to 4 packed linears that read the same input x (e.g. the
 * q/k/v or gate/up projections of a decoder layer) and share one codebook:
 * each has its own rot_scale/block, streams, scales, bias (array may be NULL),
 * output and workspace; arrays are host arrays of n_linears entries.
 * No reference counterpart: the reference calls PackedTCQLinear.forward once
 * per projection (turbopress/runtime.py:304-334); this entry point serves the
 * same calls with one launch. */
int tp_packed_linear_forward_group(int n_linears, const uint16_t* x, int64_t ldx,
                                   int64_t batch, const uint16_t* const* rot_scales,
                                   const int64_t* blocks, const uint8_t* const* path_tiled,
                                   const uint8_t* const* member_tiled,
                                   const uint16_t* const* scales, const uint16_t* codebook,
                                   const uint16_t* const* biases, const int64_t* ns,
                                   int64_t d, int bits, int n_states, uint16_t* const* ys,
                                   const int64_t* ldys, void* const* workspaces,
                                   const int64_t* workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Decode-step stack: every packed linear of a step in one persistent launch
 * ------------------------------------------------------------------------- */

/* One linear of a stack (host struct; pointers are device pointers). */
typedef struct tp_stack_linear {
  const uint8_t* path_tiled;    /* device layout, from tp_retile */
  const uint8_t* member_tiled;
  const uint16_t* x;            /* fp16 [batch, ldx] input of this linear (ldx, d multiples of 4) */
  int64_t ldx;
  const uint16_t* rot_scale;    /* fp16 [d] */
  int64_t block;                /* Hadamard block */
  const uint16_t* scales;       /* fp16 [n] */
  const uint16_t* bias;         /* fp16 [n] or NULL */
  uint16_t* y;                  /* fp16 [batch, ldy] output */
  int64_t ldy;
  int64_t n, d;
  int32_t phase;                /* dependency phase: 0 for the first linear, then equal to or one
                                   above the previous linear's (no empty phase in between) */
  int32_t reserved;
} tp_stack_linear;

/* Bytes of the device plan of these linears at this batch (0 when invalid):
 * descriptors, schedules, counters and the buffer of rotated activations
 * (batch * ceil(d/256)*256 fp16 per linear).  A plan holds 1..65536
 * linears of at most 2^21 rows each, in at most 4096 phases.  Host only. */
int64_t tp_stack_plan_bytes(const tp_stack_linear* linears, int n_linears, int bits, int64_t batch);

/* Validate the linears and write the plan (descriptors, block prefix sums,
 * phase tables, zeroed counters, batch in [1, 32]) into `plan` (device
 * memory, 256-byte aligned) with a blocking copy.  Setup call, not capturable.
 * bits in {2, 3, 4}.
 * No reference counterpart: the reference has no step-level executor; this
 * serves the decode step of scripts/graph_decode_bench.py:70-118. */
int tp_stack_plan_init(const tp_stack_linear* linears, int n_linears, int bits,
                       int64_t batch, void* plan, int64_t plan_bytes);

/* Run every linear of the plan (y = PackedTCQLinear.forward(x) for each, as
 * tp_packed_linear_forward computes it): one small launch rotates every
 * input into the plan's z buffer and ONE persistent launch runs all GEMVs
 * (batch <= 4: the slot kernel; 5..32: the wide kernel).  With
 * ordered != 0 a linear of phase p starts only after all linears of phase
 * p-1 finished (their y stores complete).  Ordering schedules work; it does
 * not pass data: every input is rotated by the first launch, before any
 * phase runs, so a phase cannot consume an earlier phase's outputs within
 * one run.  The plan's counters return to zero after each run, so one
 * plan serves any number of runs or graph replays on one stream (runs that
 * overlap on one plan race).  Sizes are read from the plan; `batch` (the
 * plan's batch) and total_blocks (tp_stack_plan_blocks) only size the launch.
 * A launch whose batch tiles cannot hold the plan's batch sets error 2 and
 * does nothing.  The codebook must be 4-byte aligned (TP_ERR_MISALIGNED
 * otherwise). */
int tp_stack_run(void* plan, int64_t batch, const uint16_t* codebook, int bits,
                 int n_states, int ordered, int64_t total_blocks, void* stream);

/* The two launches of tp_stack_run, for callers that schedule them apart:
 * tp_stack_rotate fills the plan's z buffer from the current inputs;
 * tp_stack_gemv runs the GEMVs from it.  A tp_stack_gemv run after new
 * inputs were written needs a tp_stack_rotate in between on the same
 * stream. */
int tp_stack_rotate(void* plan, int64_t batch, void* stream);
int tp_stack_gemv(void* plan, int64_t batch, const uint16_t* codebook, int bits,
                  int n_states, int ordered, int64_t total_blocks, void* stream);

/* Work blocks of a stack of linears with the given (n) sizes: sum of
 * ceil(ceil(n/16)/8).  Host only. */
int64_t tp_stack_plan_blocks(const int64_t* ns, int n_linears);

/* Copy the plan's error flag (1 = a phase wait timed out, 2 = batch mismatch) to *error_out
 * (blocking).  Not capturable. */
int tp_stack_error(const void* plan, int* error_out);

/* Decode the device layout through the same decode path the tiled GEMV uses:
 * w[r, c] = fp16(f32(codebook[level]) * f32(scales[r])), fp16 [n, out_stride].
 * bits in {2, 3, 4}.  The bit-exact check of the bandwidth path.
 * Replaces turbopress/runtime.py:291-301 (decode_rows) for this layout. */
int tp_decode_tiled(const uint8_t* path_tiled, const uint8_t* member_tiled,
                    const uint16_t* scales, const uint16_t* codebook,
                    int64_t n, int64_t d, int bits, int n_states,
                    uint16_t* w_out, int64_t out_stride, void* stream);

/* ---------------------------------------------------------------------------
 * TCQ encoder (compress time)
 * ------------------------------------------------------------------------- */

/* Workspace of tp_tcq_viterbi: one 64-bit branch-decision word per column
 * and row (n * d * 8 bytes).  Host only. */
int64_t tp_viterbi_workspace_bytes(int64_t n, int64_t d);

/* Minimum-distortion trellis path of every row of z (fp32 [n, ldz], d
 * columns used) against the doubled codebook (fp32 [2^(bits+1)], each subset
 * codebook[j::4] ascending): replaces `_viterbi` (turbopress/trellis.py:
 * 111-179; pipeline.py:209-276's copy).  Same fp32 arithmetic and
 * tie-breaking: nearest member = number of subset midpoints strictly below z
 * (torch.bucketize), branch 1 only if strictly cheaper, end state = first
 * state of minimum metric.  Each row starts in start_state[row] (NULL:
 * state 0).  Outputs uint8 [n, d] level codes (member * 4 + subset), path
 * bits and member codes, and int32 end_state[n] (may be NULL).  bits in
 * 1..4, n_states in {4, 8, 16, 64}; workspace of
 * tp_viterbi_workspace_bytes(n, d), 8-byte aligned, contents irrelevant. */
int tp_tcq_viterbi(const float* z, int64_t ldz, int64_t n, int64_t d, const float* codebook, int bits,
                   int n_states, const int32_t* start_state, uint8_t* level_codes, uint8_t* path_bits,
                   uint8_t* member_codes, int32_t* end_state, void* workspace, int64_t workspace_bytes,
                   void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TURBOPRESS_AMD_H */
