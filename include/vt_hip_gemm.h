/*
 * vt_hip_gemm.h -- C ABI of libvt_hip_gemm.so, the MI355X (gfx950) exact
 * int8 x int8 -> int32 GEMM behind the `hip_gemm` specialization.
 *
 * Contract (same as the reference's Gemmini GEMM, extended by an explicit
 * initial partial sum):
 *     C[b][i][j] = D[b][i][j] + sum_t A[b][i][t] * B[b][t][j]      (D optional)
 * with int32 accumulation modulo 2^32 (VeriTac/Gemmini/Word.lean:11, :31) over
 * row-major operands A[i*lda+t], B[t*ldb+j], C[i*ldc+j]
 * (VeriTac/Gemmini/Semantics.lean:76-77, specializations/gemmini_gemm/
 * backend.py:569-580). Inside the reference's legality bound
 * k*16384 <= 2^31-1 (VeriTac/Gemmini/Plan.lean:86-92) plus |D| the result is
 * the exact integer product; outside it the result is the wrapped int32 sum,
 * which is what the Lean model's signed32 accumulator computes.
 *
 * The reference has no FFI for this path: its specialization API is Python
 * (specializations/gemmini_gemm/backend.py, specializations/cpu_gemm/
 * runner.py) and its native layer is emitted C run as a subprocess
 * (cpu_gemm/runner.py:65-108) or Gemmini command streams on Spike. This
 * header replaces that native execution layer; the Python specialization
 * (specializations/hip_gemm/backend.py) binds it with ctypes.
 *
 * Conventions:
 *   - every function returns 0 (VT_OK) or a negative VT_E* code; the message
 *     of the last failure on the calling thread is vt_last_error();
 *   - argument and shape validation happens on the host before any device
 *     call, so invalid input never reaches a kernel;
 *   - pointers are device pointers owned by the caller (borrowed for the
 *     call); the library never allocates or frees caller buffers;
 *   - `stream` is a hipStream_t (NULL = the default stream); work is
 *     enqueued asynchronously on it.
 */
#ifndef VT_HIP_GEMM_H
#define VT_HIP_GEMM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VT_ABI_VERSION 7

/* Status codes. */
#define VT_OK 0
#define VT_EINVAL (-1)        /* null pointer, negative size, bad stride     */
#define VT_EUNSUPPORTED (-2)  /* variant cannot run this shape / alignment   */
#define VT_EHIP (-3)          /* HIP runtime error (launch, allocation, ...) */
#define VT_ENODEV (-4)        /* no HIP device, or the device is not gfx950  */

/* Kernel variants. VT_VARIANT_AUTO picks one from the shape. */
#define VT_VARIANT_AUTO 0
#define VT_VARIANT_MFMA_256x256 1  /* compute-bound: 256x256 tile, 4 waves;
                                      M, N >= 256 with K % 256 == 0 and
                                      16-byte C / D rows on
                                      v_mfma_i32_16x16x64_i8 (C stored
                                      through LDS), else
                                      v_mfma_i32_32x32x32_i8; a partial
                                      last tile row or column ends at M or
                                      N (stores masked to the elements no
                                      other tile writes), or, when it saves
                                      a round of tiles, the rows (columns)
                                      past whole tiles run on 128x128 tiles   */
#define VT_VARIANT_MFMA_128x128 2  /* 128x128 tile, 4 waves,
                                      v_mfma_i32_32x32x32_i8; 64x128 tiles
                                      with row-major B when that gives at
                                      most 256 workgroups over at most 2048
                                      of K (1024 per K slice), 64x64 tiles
                                      when those do as well                   */
#define VT_VARIANT_SKINNY 3        /* M <= 64 decode shapes: B streamed once,
                                      v_mfma_i32_16x16x64_i8, K split         */
#define VT_VARIANT_GENERIC 4       /* any shape/stride/alignment, VALU        */
#define VT_VARIANT_MFMA_256x128 5  /* 256x128 tile, 4 waves; M >= 256, N >= 128,
                                      K % 256 == 0 with 16-byte aligned C, D
                                      run persistently (one workgroup per CU) */
#define VT_VARIANT_PADDED 6        /* any shape: A and B copied with K and N
                                      zero-padded to multiples of 16, run on
                                      the MFMA / skinny kernels, C copied out
                                      (plus D)                                */
#define VT_VARIANT_COUNT 7

/*
 * vt_gemm_i8 -- batched exact int8 GEMM.
 *
 * Replaces the execution of one GEMM by the reference's specializations:
 * `run_commands` (specializations/gemmini_gemm/backend.py:433-562) and the
 * emitted scalar kernel `veritac_scalar_ref` (backend.py:712-720) for the
 * Gemmini contract, and the emitted loop nest timed by `benchmark_matmul`
 * (specializations/cpu_gemm/runner.py:111-232). Batched B-reuse
 * (specializations/gemmini_gemm/lowering.py:18-40) is stride_b == 0.
 *
 *   A  int8  [batch][M][lda]  (stride_a elements between batches)
 *   B  int8  [batch][K][ldb]  (stride_b elements; 0 = one B shared by all)
 *   D  int32 [batch][M][ldd]  initial partial sum, or NULL for zero
 *   C  int32 [batch][M][ldc]  output (may alias D exactly: in-place C += A.B)
 *   M, N, K >= 0 (M == 0 or N == 0: nothing to do; K == 0: C = D or 0)
 *   lda >= K, ldb >= N, ldd >= N, ldc >= N
 *   variant: VT_VARIANT_*; k_split: K slices for VT_VARIANT_SKINNY
 *            (0 = choose automatically; ignored by other variants)
 *
 * The MFMA and skinny variants need N % 16 == 0, K % 16 == 0, lda and ldb
 * multiples of 16 and 16-byte-aligned A and B; an explicit one returns
 * VT_EUNSUPPORTED otherwise. For such shapes VT_VARIANT_AUTO picks
 * VT_VARIANT_PADDED from 3 * 2^24 multiply-adds on (M, N + 15, K + 15 < 2^30,
 * batch <= 65535) and VT_VARIANT_GENERIC below. VT_VARIANT_PADDED copies
 * the operands the vector variants cannot read as they are, zero padded, to
 * a workspace the library allocates once per (device, stream) and grows as
 * needed; when N % 16 == 0 the product writes C directly. For aligned
 * shapes VT_VARIANT_AUTO picks VT_VARIANT_SKINNY for M <= 16, and for
 * M <= 64 when K >= 512 and ceil(N / 128) * batch < 256 (the skinny kernel
 * runs 1, 2 or 4 row blocks of 16 over one stream of B), VT_VARIANT_GENERIC when K <= 64 and
 * M * N * K * batch <= 2^20 (faster than any MFMA launch there), and an MFMA
 * variant otherwise. The MFMA variants
 * address each tile from a 64-bit base with 32-bit offsets inside it, so
 * they need 256 * lda and 64 * ldb below 2^32 (K < 2^24 for contiguous A):
 * VT_VARIANT_AUTO picks VT_VARIANT_GENERIC beyond that, and an explicit MFMA
 * variant returns VT_EUNSUPPORTED.
 *
 * Workspace: the skinny variant's K-split partial sums and the padded
 * variant's copies live in workspaces the library allocates per (device,
 * stream, kind). With a K split over at most 16 rows the decode kernels
 * (row-major or packed B) finish the slices' sums themselves (when the
 * split's arrival count fits the word), through one 8-byte finishing word
 * per two output elements in a
 * workspace of its own kind that is zeroed when it is allocated and that
 * every call leaves zero (no second launch, and never more bytes than the
 * partial sums). A workspace only grows, and a
 * superseded one is kept (not freed) until the process ends, so a HIP graph
 * captured with an earlier workspace stays valid. Growth is refused while
 * the stream is being captured: a call that needs more workspace than its
 * stream has returns VT_EUNSUPPORTED during capture, so make the same calls
 * once on the stream before capturing (vt_gemm_check reports the bytes a
 * call takes from vt_gemm_i8_noalloc's array, which bounds what it takes
 * from a stream's workspaces). Graphs captured on one stream use that
 * stream's workspaces: replay them in order on that stream (or with the same
 * ordering against it), never two at once. Overlapping launches on one
 * workspace race, and racing finishing words can stay nonzero and spoil the
 * later calls that use them.
 *
 * Sizes up to 2^40, leading dimensions up to 2^40, batch up to 2^31, batch
 * strides up to 2^56, and every operand's byte extent below 2^56. C may not
 * share memory with A, B or D, except D == C with ldd == ldc and (batch > 1)
 * stride_d == stride_c, which is in place. Anything else returns VT_EINVAL
 * before the device is touched.
 */
int vt_gemm_i8(const int8_t *A, const int8_t *B, const int32_t *D, int32_t *C,
               int64_t M, int64_t N, int64_t K,
               int64_t lda, int64_t ldb, int64_t ldd, int64_t ldc,
               int64_t batch, int64_t stride_a, int64_t stride_b,
               int64_t stride_d, int64_t stride_c,
               int32_t variant, int32_t k_split, void *stream);

/*
 * vt_gemm_i8_noalloc -- vt_gemm_i8 without any allocation.
 *
 * No counterpart in the reference. For callers that cannot allocate device
 * memory during the call: code under HIP graph capture (including a first
 * call on a stream), tight serving loops, harnesses that forbid hipMalloc.
 * Same arguments, checks and results as vt_gemm_i8, and it calls no
 * hipMalloc, hipFree or other allocating routine: the K-split partial sums
 * and padded copies that vt_gemm_i8 keeps in per-stream workspaces live in
 * one static device array of VT_NOALLOC_SCRATCH_BYTES (32 MiB) per device,
 * held until the process ends. A call that needs more (vt_gemm_check
 * reports the bytes) returns VT_EUNSUPPORTED before anything is launched.
 * Every call on a device shares that device's array and nothing in it needs
 * clearing between calls (each call writes all the scratch it reads), so
 * calls that overlap on one device -- on different streams, or from
 * different threads without ordering -- race: order them on one stream.
 */
#define VT_NOALLOC_SCRATCH_BYTES (32 << 20)
int vt_gemm_i8_noalloc(const int8_t *A, const int8_t *B, const int32_t *D,
                       int32_t *C, int64_t M, int64_t N, int64_t K,
                       int64_t lda, int64_t ldb, int64_t ldd, int64_t ldc,
                       int64_t batch, int64_t stride_a, int64_t stride_b,
                       int64_t stride_d, int64_t stride_c,
                       int32_t variant, int32_t k_split, void *stream);

/*
 * vt_gemm_check -- the host-side acceptance check of vt_gemm_i8, without
 * operands: returns VT_OK when vt_gemm_i8 would accept a call with these
 * sizes, strides, D present or not (has_d), variant and k_split on distinct
 * 16-byte aligned buffers, else the VT_E* code vt_gemm_i8 would return, with
 * the reason in vt_last_error(). On VT_OK it stores the variant and K split
 * that would run (VT_VARIANT_AUTO resolved; VT_VARIANT_AUTO and 0 when there
 * is nothing to compute) and the bytes of workspace the call takes. Any
 * output pointer may be NULL. No device call: it runs without a GPU.
 *
 * The counterpart of the reference's external plan checker `gemmini_check`
 * (specializations/gemmini_gemm/backend.py:164-196), whose verdict
 * `optimize` records per candidate as check{accepted, reason}
 * (backend.py:1083-1091).
 */
int vt_gemm_check(int64_t M, int64_t N, int64_t K,
                  int64_t lda, int64_t ldb, int64_t ldd, int64_t ldc,
                  int64_t batch, int64_t stride_a, int64_t stride_b,
                  int64_t stride_d, int64_t stride_c,
                  int32_t has_d, int32_t variant, int32_t k_split,
                  int32_t *variant_out, int32_t *k_split_out,
                  int64_t *scratch_bytes_out);

/* vt_gemm_select flags. */
#define VT_SELECT_ALIGNED 1   /* A and B 16-byte aligned (else: unaligned) */
#define VT_SELECT_B_SHARED 2  /* batch > 1 shares one B (stride_b == 0)    */

/*
 * vt_gemm_select -- the variant (and K split) VT_VARIANT_AUTO would launch
 * for contiguous operands (stride_a = M*lda, stride_c = M*N, stride_b 0 with
 * VT_SELECT_B_SHARED else K*ldb). Mirrors the reference's candidate
 * selection (`optimize`, backend.py:1072-1093) at the native layer; no
 * device call.
 */
int vt_gemm_select(int64_t M, int64_t N, int64_t K, int64_t batch,
                   int64_t lda, int64_t ldb, int32_t flags,
                   int32_t *variant_out, int32_t *k_split_out);

/*
 * vt_variant_info -- static resources of one variant: tile sizes, threads per
 * workgroup, LDS bytes per workgroup. Mirrors `required_resources`
 * (backend.py:97-104). No device call. For the MFMA variants the LDS is that
 * of their tile kernel (three 64-deep slice buffers of A and B); the
 * persistent 256x256 kernels, one workgroup per CU, take 160 KiB (K % 256 == 0
 * with 16-byte C and D rows) or 128 KiB, and so does the persistent form of
 * 256x128 (160 KiB; M >= 256, N >= 128, K % 256 == 0, 16-byte C and D rows). The
 * skinny figure excludes the A slice, which depends on K and the split.
 */
int vt_variant_info(int32_t variant, int32_t *tile_m, int32_t *tile_n,
                    int32_t *tile_k, int32_t *threads, int32_t *lds_bytes);

/* Name of a variant ("mfma_256x256", ...) or NULL for an unknown id. */
const char *vt_variant_name(int32_t variant);

/* Message of the last failure on the calling thread ("" if none). */
const char *vt_last_error(void);

/* hipStreamSynchronize(stream), reporting asynchronous kernel errors. */
int vt_sync(void *stream);

/* Number of usable gfx950 devices (0 if none); no error on a GPU-less host. */
int vt_device_count(void);

/* VT_ABI_VERSION of the loaded library. */
int vt_abi_version(void);

/*
 * Gemmini command-stream replay.
 *
 * vt_replay_i8 executes a weight-stationary Gemmini command stream (the
 * `commands` of a veritac_program_request_v1, specializations/gemmini_gemm/
 * backend.py:891-936) on the GPU with the semantics of the reference's
 * interpreter `run_commands` (backend.py:433-562): a scratchpad of int8 rows,
 * an accumulator of int32 rows, mvin / compute / mvout tile moves, overwrite
 * or accumulate into the accumulator, and rejection of int32 overflow. It
 * replaces that interpreter's execution step; the stream's static checks
 * (configuration order, address spaces, initialised reads, fences, every
 * output written) run on the host first (specializations/hip_gemm/replay.py),
 * which lowers the stream to the tile program below.
 *
 * program: device pointer to n_ops operations of 8 int32 words each,
 *   { VT_REPLAY_MVIN,    buf (0 = A, 1 = B), offset, row stride, scratchpad row, -, -, index }
 *   { VT_REPLAY_LATCH_B, scratchpad row, -, -, -, -, -, index }
 *   { VT_REPLAY_COMPUTE, A scratchpad row, accumulator row, accumulate (0/1), -, -, -, index }
 *   { VT_REPLAY_MVOUT,   accumulator row, C offset, C row stride, -, -, -, index }
 *   (offsets and strides in elements; every tile is 16 x 16; `index` is the
 *   position of the originating command, reported on failure).
 * A int8 [m*k], B int8 [k*n], C int32 [m*n]: device pointers, row-major.
 * status: device pointer to 4 int32 words the kernel fills with
 *   { VT_REPLAY_STATUS_*, index, row, column } of the first failure, or zeros.
 * Every operand address is bounds-checked on the device as well; an
 * operation outside m, n, k or the scratchpad / accumulator sizes stops the
 * replay with VT_REPLAY_STATUS_RANGE instead of touching memory.
 * The scratchpad (16 bytes per row) and accumulator (64 bytes per row) live
 * in LDS: scratchpad_rows * 16 + accumulator_rows * 64 <= 152 KiB.
 */
#define VT_REPLAY_MVIN 1
#define VT_REPLAY_LATCH_B 2
#define VT_REPLAY_COMPUTE 3
#define VT_REPLAY_MVOUT 4
#define VT_REPLAY_STATUS_OK 0
#define VT_REPLAY_STATUS_OVERFLOW 1   /* int32 accumulator overflow         */
#define VT_REPLAY_STATUS_RANGE 2      /* operand outside the declared sizes */
#define VT_REPLAY_STATUS_OPCODE 3     /* unknown operation                  */

int vt_replay_i8(const int32_t *program, int64_t n_ops, const int8_t *A, const int8_t *B,
                 int32_t *C, int64_t m, int64_t n, int64_t k, int64_t scratchpad_rows,
                 int64_t accumulator_rows, int32_t *status, void *stream);

/*
 * Device query for hardware profiles.
 *
 * vt_device_query fills `info` with what the HIP runtime reports for one
 * device. It replaces the driver probe of the reference's hardware profile
 * (Hardware/profile.py:180-265, `_probe_cuda`: cuDeviceGetName,
 * cuDeviceGetAttribute, cuDeviceTotalMem_v2), which has no ROCm backend; the
 * Python side (specializations/hip_gemm/provenance.py) normalises it into the
 * same schema_version 1 profile. `supported` is 1 when the device's ISA is
 * the one this library's code objects are built for (code_object_arch), the
 * condition under which every other entry point runs on it.
 *
 * device: device ordinal, or -1 for the calling thread's current device.
 * info_size: sizeof(vt_device_info) as the caller sees it; a mismatch
 *   returns VT_EINVAL, so a binding built against another layout fails
 *   instead of reading past the structure.
 * Returns VT_ENODEV on a host without HIP devices, VT_EINVAL for a bad
 * ordinal or pointer, VT_EHIP if the runtime refuses the query.
 */
typedef struct vt_device_info {
  char name[256];                  /* marketing name ("AMD Instinct MI355X")   */
  char arch[256];                  /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  char code_object_arch[32];       /* ISA the library was compiled for        */
  int64_t total_memory_bytes;      /* HBM capacity                             */
  int64_t l2_cache_bytes;          /* L2 as the runtime reports it (per XCD)  */
  int64_t lds_per_workgroup_bytes; /* largest LDS allocation of one workgroup */
  int64_t lds_per_cu_bytes;        /* LDS of one compute unit                  */
  int32_t compute_units;
  int32_t wavefront_size;
  int32_t max_threads_per_workgroup;
  int32_t max_clock_khz;           /* peak engine clock                        */
  int32_t memory_clock_khz;
  int32_t memory_bus_width_bits;
  int32_t pci_domain;
  int32_t pci_bus;
  int32_t pci_device;
  int32_t hip_runtime_version;     /* hipRuntimeGetVersion                     */
  int32_t hip_driver_version;      /* hipDriverGetVersion                      */
  int32_t supported;               /* 1: arch matches code_object_arch         */
} vt_device_info;

int vt_device_query(int32_t device, vt_device_info *info, int64_t info_size);

/*
 * Packed-B decode path.
 *
 * A decode-shaped GEMM (M <= 64 rows of activations against K x N int8
 * weights) is bound by streaming B from HBM once. Row-major B makes the
 * kernel transpose it through LDS and split K across workgroups to reach
 * enough memory parallelism, which costs a second reduction launch. When the
 * same weights serve many calls, pack them once into the layout below and
 * call vt_gemm_i8_packed: every wave then loads its MFMA operand straight
 * from HBM in 1 KiB coalesced pieces, K is not split, and the result is the
 * same C = D + A.B as vt_gemm_i8, bit for bit.
 *
 * The reference keeps weights row-major and has no packed format; this is an
 * MI355X layout for the skinny shape of the reference's GEMM contract
 * (VeriTac/Gemmini/Semantics.lean:76-77), with the same arithmetic.
 *
 * Layout: Kp = K rounded up to a multiple of 64, kbt = Kp / 64. For each
 * 16-column block nb (0 <= nb < N/16) and 64-row block kb (0 <= kb < kbt) a
 * 1024-byte tile at byte offset (nb * kbt + kb) * 1024 holds, at tile byte
 * l * 16 + i (l = 0..63, i = 0..15),
 *     B[kb*64 + 16*(l/16) + i][nb*16 + l%16]     (0 for rows >= K).
 * That is the B operand of v_mfma_i32_16x16x64_i8 for lane l. One packed B
 * takes N * Kp bytes; every 16-column block is contiguous over K.
 */

/* Bytes of one packed B (N * Kp), or a negative VT_E* code (N % 16 != 0,
 * negative or >= 2^30 sizes). No device call. */
int64_t vt_packed_b_size(int64_t K, int64_t N);

/*
 * vt_pack_b_i8 -- row-major B int8 [batch][K][ldb] -> packed B
 * [batch][vt_packed_b_size(K, N)] (stride_b / stride_bp bytes between
 * batches). Needs N % 16 == 0, ldb and strides multiples of 16, 16-byte
 * aligned B and Bp. Asynchronous on `stream`, like vt_gemm_i8.
 */
int vt_pack_b_i8(const int8_t *B, int8_t *Bp, int64_t K, int64_t N, int64_t ldb,
                 int64_t batch, int64_t stride_b, int64_t stride_bp, void *stream);

/*
 * vt_gemm_i8_packed -- C = D + A.B with B packed by vt_pack_b_i8.
 *
 * Same contract, argument meaning and error behaviour as vt_gemm_i8
 * (which replaces specializations/gemmini_gemm/backend.py:433-562 /
 * :712-720 execution), with B given packed: Bp [batch][packed size],
 * stride_bp 0 = one packed B shared by every batch. Needs N % 16 == 0,
 * K % 16 == 0, lda and strides multiples of 16, 16-byte aligned A and Bp.
 * Same extent bounds and overlap refusals as vt_gemm_i8 (Bp counts as
 * batch blocks of vt_packed_b_size bytes; vt_pack_b_i8 likewise refuses a Bp
 * that overlaps B). Any M. The rows run on three kernels:
 *   - whole 256-row tiles, when N % 256 == 0, K % 64 == 0 and there are at
 *     least 128 such tiles over all batches: the persistent 256x256 MFMA
 *     kernels of vt_gemm_i8 (16x16x64 when K % 256 == 0, else 32x32x32),
 *     which read each B operand with one ds_read_b128 (a 1 KiB tile holds
 *     16 consecutive k per lane, the k order of the A operand); below that,
 *     every row on their 256x128 form when there are more than 128 but at
 *     most 256 of its tiles (M >= 256, N % 128 == 0, K >= 1024 with
 *     K % 256 == 0);
 *   - more than 64 remaining rows: 128 x 128 MFMA tiles reading the packed
 *     tiles the same way, K split into up to 16 slices (a second kernel adds
 *     them) when fewer than 64 tiles would run, as vt_gemm_i8 does;
 *   - up to 64 rows (or tiles whose offsets exceed 32 bits): groups of up to
 *     64 rows, each group streaming B once for its 1, 2 or 4 row blocks of
 *     16. Columns go to workgroups in groups of 8-column half blocks: whole
 *     groups of four 16-column blocks when N gives 192 or more of them, else
 *     smaller groups, about one per CU.
 * k_split: workgroups along K for the groups of up to 64 rows (0 =
 * automatic: 1 unless even half-block groups are too few, else a split whose
 * partial sums are finished in the kernel up to 16 rows, through the
 * finishing words described under Workspace, or added by a second kernel);
 * the tile kernels choose their own.
 */
int vt_gemm_i8_packed(const int8_t *A, const int8_t *Bp, const int32_t *D, int32_t *C,
                      int64_t M, int64_t N, int64_t K,
                      int64_t lda, int64_t ldd, int64_t ldc, int64_t batch,
                      int64_t stride_a, int64_t stride_bp, int64_t stride_d,
                      int64_t stride_c, int32_t k_split, void *stream);

/*
 * Run-time compiled loop-nest kernels.
 *
 * The reference turns a loop nest (its `Stmt` JSON, README.md:456-503) into
 * C with emit_c.py (specializations/cpu_gemm/emit_c.py:83-155) and runs it
 * through gcc as a subprocess (specializations/cpu_gemm/runner.py:65-108).
 * Here the Python emitter (specializations/hip_gemm/loopnest.py) writes a
 * HIP kernel instead, and these entry points replace the gcc + subprocess
 * step: hipRTC compiles the source for gfx950 in process, and the kernel is
 * launched on the caller's stream.
 *
 * vt_rtc_compile: compile `source`, which must define
 *   extern "C" __global__ void <kernel_name>(...); no device is needed.
 *   On a compiler error it returns VT_EINVAL and vt_last_error() holds the
 *   start of the compiler log. *out is a library-owned handle, freed by
 *   vt_rtc_release.
 * vt_rtc_code_size: bytes of the compiled code object (negative: VT_E*).
 * vt_rtc_launch: load the code object on the current device (once) and
 *   launch grid x block threads; args[i] points at the value of the kernel's
 *   i-th parameter (hipModuleLaunchKernel's convention) and must match the
 *   kernel's parameter list.
 */
typedef struct vt_rtc_program vt_rtc_program;

int vt_rtc_compile(const char *source, const char *kernel_name, vt_rtc_program **out);
int64_t vt_rtc_code_size(const vt_rtc_program *program);
int vt_rtc_launch(vt_rtc_program *program, uint32_t grid_x, uint32_t grid_y, uint32_t grid_z,
                  uint32_t block_x, uint32_t block_y, uint32_t block_z, void **args,
                  void *stream);
void vt_rtc_release(vt_rtc_program *program);

#ifdef __cplusplus
}
#endif

#endif /* VT_HIP_GEMM_H */
