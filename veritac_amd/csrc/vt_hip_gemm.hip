// vt_hip_gemm.hip -- exact int8 x int8 -> int32 GEMM for MI355X (gfx950).
//
// Contract: C = D + A.B with int32 accumulation mod 2^32 over row-major
// operands (VeriTac/Gemmini/Semantics.lean:76-77, Word.lean:31; the reference
// oracles are specializations/gemmini_gemm/backend.py:569-580 and the emitted
// `veritac_scalar_ref`, backend.py:712-720). Any K split, tile order or MFMA
// k-ordering gives the same int32 result because addition mod 2^32 is
// associative and commutative (GemminiExact.lean:16-30), which is what every
// kernel here relies on.
//
// Kernels
//   gemm_dma16_kernel  256x256 tiles with M, N >= 256, K % 256 == 0 and
//       16-byte C (and D) rows, with or without D, row-major or packed B (the
//       8192^3 case and config 3). When M or N is not whole tiles, the last
//       tile row or column starts at M - 256 or N - 256 and leaves the rows
//       and columns it shares with its neighbour to the neighbour's stores.
//       Persistent: one workgroup
//       per CU walks its tiles in XCD-contiguous order; k slices go global ->
//       LDS by direct-to-LDS DMA (global_load_lds_dwordx4) into four stages,
//       three slices ahead, and the slice stream runs across tile
//       boundaries. Each wave's 128x128 block is 8 x 8 v_mfma_i32_16x16x64_i8
//       accumulators (half the accumulator traffic per multiply-add of the
//       32x32x32 form, so more work per joule under the board's power limit);
//       the MFMA, fragment-read and DMA instructions follow an explicit
//       per-slot schedule. C leaves through an 8 KB LDS strip per wave as
//       whole 512-byte row segments; without D, six of a tile's eight strips
//       go out during its last k step.
//   gemm_dma_kernel  the same on 4 x 4 v_mfma_i32_32x32x32_i8 accumulators
//       (4-byte C stores), for the problems the 16x16x64 kernel does not
//       take: K a multiple of 64 but not of 256, or C / D rows it cannot
//       store as 16-byte pieces.
//   gemm_mfma_kernel<BM,BN>  every other compute-bound case. 256 threads = 4
//       waves in a 2x2 grid, each wave owns a (BM/2)x(BN/2) block of 32x32
//       accumulators fed by v_mfma_i32_32x32x32_i8. A/B k-slices of 64 bytes
//       are staged global -> VGPR -> LDS (three LDS buffers, next slices'
//       global loads in flight during the MFMAs). A is stored [m][k] and read
//       with ds_read_b128; B stays row-major [k][n] in LDS and is read into
//       the MFMA operand layout with ds_read_b64_tr_b8 (gfx950's transposing
//       LDS read), so B is never transposed in memory. 16-byte chunks are
//       XOR-swizzled so the LDS accesses are bank-conflict free. Workgroup ids
//       are remapped so consecutive tiles share an XCD (and its L2), then
//       grouped along M. A K of at most 128 runs the SHORT instantiation,
//       which fetches its two slices in one round trip.
//   skinny_kernel<NB>  M <= 64 (decode and small batches). Bandwidth-bound:
//       each workgroup streams an NB-column slab of B exactly once over a K
//       slice with non-temporal loads, U stages of 64 rows in flight in
//       registers, LDS double buffer, the A slice resident in LDS,
//       v_mfma_i32_16x16x64_i8 over 1, 2 or 4 row blocks of 16 (M padded up).
//       K slices write int32 partials to a workspace and skinny_reduce_kernel,
//       next on the same stream, adds them (and D); up to 16 rows the kernel
//       finishes them itself through one 64-bit word per two output elements.
//   generic_kernel  any shape, stride or alignment; one thread per output,
//       int32 VALU. Used where the vector kernels' alignment rules fail.
//
// Tails: rows of A past M and columns of B past N are read from clamped (valid)
// addresses and their outputs are never stored; k past K reads A as zero, so
// the clamped B rows there contribute nothing.

#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "vt_hip_gemm.h"

// Scratch memory of vt_gemm_i8_noalloc: K-split partial sums and padded
// operand copies of one call, in consecutive 256-byte aligned pieces. Each
// device holds its own copy for the life of the process; host code reaches
// it only through the address hipGetSymbolAddress returns on that device
// (DeviceState::scratch), never through this name.
static __device__ __align__(256) int8_t scratch[32 << 20];

typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
#define LDS_AS __attribute__((address_space(3)))

namespace {

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------

// Workgroup barrier that orders LDS only: waits for this wave's LDS accesses
// (lgkmcnt) but leaves global loads in flight across the barrier.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ v4i ld_lds_b128(const int8_t *base, int off) {
  return *(const LDS_AS v4i *)((const LDS_AS int8_t *)base + off);
}

__device__ __forceinline__ void st_lds_b128(int8_t *base, int off, v4i v) {
  *(LDS_AS v4i *)((LDS_AS int8_t *)base + off) = v;
}

// ds_read_b64_tr_b8: within each 16-lane group, lane j supplies the address of
// the 8 bytes (row j/2, column half j%2) of an 8-row x 16-column byte block and
// receives column j of that block (byte r = row r).
__device__ __forceinline__ v2i ld_lds_tr8(const int8_t *base, int off) {
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32(
      (LDS_AS v2i *)((LDS_AS int8_t *)base + off));
}

__device__ __forceinline__ int32_t add_wrap(int32_t a, int32_t b) {
  return (int32_t)((uint32_t)a + (uint32_t)b);
}

// LDS swizzles. gfx950's LDS has 64 banks of 4 bytes (256 bytes per cycle).
// Measured lane grouping (one bank cycle each, conflict-free only if the
// group's addresses fall on distinct banks):
//   ds_read_b128: four groups of 16 lanes, lane L in group
//     parity((L >> 2) & 7) + 2 * (L >> 5), e.g. {0-3, 12-15, 20-27};
//   ds_read_b64 / ds_read_b64_tr_b8: lanes 0-31 and lanes 32-63.
// The swizzles below keep every group on distinct banks for the access
// patterns of the kernels:
//   A slice [m][64 B], ds_read_b128 of one 16-byte chunk from 32 consecutive
//     rows: chunk c of row r is stored at c ^ ((r >> 2) & 3), which gives the
//     four rows of equal r % 4 within each lane group four distinct chunks;
//   B slice [k][n], ds_read_b64_tr_b8 of 8 consecutive rows by 16 lanes, two
//     16-lane groups reading adjacent chunks (c, c ^ 1) of the same rows:
//     chunk c of row r is stored at c ^ b_swz(r).
template <int CHUNKS>
__device__ __forceinline__ int b_swz(int row) {
  static_assert(CHUNKS >= 4, "B slice needs at least 4 chunks per row");
  if (CHUNKS >= 16) return ((row & 7) << 1) | ((row >> 2) & 1);
  if (CHUNKS == 8) return row & 7;
  return (row >> 1) & 3;
}

__device__ __forceinline__ int a_swz(int row) { return (row >> 2) & 3; }

__device__ __forceinline__ int a_off(int row, int c) {
  return row * 64 + ((c ^ a_swz(row)) << 4);
}

// Epilogue shared by the MFMA kernels. 32x32 accumulator layout: element e
// of lane l is row 8*(e/4) + 4*(l/32) + e%4 and column l%32 of the block, so
// one store instruction writes two full 128-byte row segments of C. C is
// written with non-temporal stores: every CU reaches a tile end at about the
// same time, and streaming the whole C tile out keeps that burst from
// displacing the A/B panels the L2 still serves.
//
// With D, each 32-row block first loads all of its D values and only then
// stores: C may be D itself (in place), so a D load that followed a C store
// in program order could not be moved above it, and loading per element
// would make every element wait one full memory round trip (this took an
// 8192^3 GEMM with D from ~480 to ~870 us). Each element's D is still read
// before its own C is written, and no other lane writes that element.
//
// LOWER: the tile may have been moved back to end at M or N (persistent
// kernels); rows below row_min and columns below col_min belong to the
// neighbouring tile, which stores them, so they are not stored here.
template <int MI, int NI, bool EDGE, bool HAS_D, bool LOWER = false>
__device__ __forceinline__ void store_tile(const v16i (&acc)[MI][NI], int32_t *Cb,
                                           const int32_t *Db, int64_t ldc, int64_t ldd,
                                           int row0, int col0, int M, int N, int lane,
                                           int row_min = 0, int col_min = 0) {
#pragma unroll
  for (int mi = 0; mi < MI; ++mi) {
    int32_t d[HAS_D ? NI : 1][16];
    if constexpr (HAS_D) {
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) {
        const int col = col0 + ni * 32 + (lane & 31);
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int row = row0 + mi * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
          d[ni][e] = (!EDGE || (row < M && col < N)) ? Db[(int64_t)row * ldd + col] : 0;
        }
      }
    }
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) {
      const int col = col0 + ni * 32 + (lane & 31);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = row0 + mi * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
        if ((!EDGE || (row < M && col < N)) && (!LOWER || (row >= row_min && col >= col_min))) {
          int32_t v = acc[mi][ni][e];
          if constexpr (HAS_D) v = add_wrap(v, d[ni][e]);
          __builtin_nontemporal_store(v, Cb + (int64_t)row * ldc + col);
        }
      }
    }
    // One 32-row block at a time: keeps the D loads from being hoisted for
    // the whole tile at once (they would not fit in registers).
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Initial partial sums D of one wave's tile, in the accumulator layout of
// store_tile, loaded into registers (rows or columns past M, N read 0).
template <int MI, int NI, bool EDGE>
__device__ __forceinline__ void load_d_tile(int32_t (&d)[MI][NI][16], const int32_t *Db,
                                            int64_t ldd, int row0, int col0, int M, int N,
                                            int lane) {
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) {
      const int col = col0 + ni * 32 + (lane & 31);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = row0 + mi * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
        d[mi][ni][e] = (!EDGE || (row < M && col < N)) ? Db[(int64_t)row * ldd + col] : 0;
      }
    }
}

// ---------------------------------------------------------------------------
// Compute-bound MFMA kernel
// ---------------------------------------------------------------------------

struct GemmArgs {
  const int8_t *A;
  const int8_t *B;
  const int32_t *D;
  int32_t *C;
  int64_t lda, ldb, ldd, ldc;
  int64_t sa, sb, sd, sc;
  int M, N, K;
  int tiles_m, tiles_n, group_m;
  int batch_count;   // batches (the persistent kernel walks all their tiles)
};

// EDGE: 0 full tiles; 1 M or N not a multiple of the tile (clamped source
// rows and columns, masked stores); 2 also K not a multiple of 128 (each load
// checks the K tail). The K checks sit in the k loop, so a ragged M or N
// alone does not pay for them.
//
// PACKED_B: B is in the packed layout of vt_pack_b_i8 (p.B = Bp, p.ldb = kbt,
// the 64-row blocks per 16-column block; p.sb = the packed batch stride). A
// 64-deep slice of the tile's B is then BN/16 whole 1 KB tiles, staged into
// LDS as they are, and each 32x32 B operand is one ds_read_b128 (lane l: the
// 16 k of column l % 32 that its A operand also holds). Rows past K are zero
// in the layout, so B needs no K-tail test; columns past N re-read the last
// 16-column block and are masked at the store.
template <int BM, int BN, int EDGE, bool HAS_D, bool SHORT, bool EARLY_D, bool PACKED_B = false>
__global__ __launch_bounds__(256, 1) void gemm_mfma_kernel(GemmArgs p) {
  constexpr int BK = 64;
  constexpr int WTM = BM / 2, WTN = BN / 2;   // wave tile (2x2 waves)
  constexpr int MI = WTM / 32, NI = WTN / 32; // 32x32 blocks per wave
  constexpr int BCH = BN / 16;                // 16-byte chunks per B row
  constexpr int CA = BM * (BK / 16) / 256;    // A chunks per thread per slice
  constexpr int CB = BK * BCH / 256;          // B chunks per thread per slice
  constexpr int A_BYTES = BM * BK, B_BYTES = BK * BN;
  static_assert(CA >= 1 && CB >= 1 && BCH >= 4, "tile too small");

  constexpr int NBUF = 3;                     // LDS slice buffers
  __shared__ __attribute__((aligned(16))) int8_t smem[NBUF * (A_BYTES + B_BYTES)];
  static_assert(sizeof(smem) == 3 * (BM * 64 + 64 * BN), "LDS vt_variant_info reports");
  int8_t *const As0 = smem;                  // A slice buffer b at As0 + b*A_BYTES
  int8_t *const Bs0 = smem + NBUF * A_BYTES; // B slice buffer b at Bs0 + b*B_BYTES

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // XCD-aware remap: hardware dispatches workgroup w to XCD w % 8; give each
  // XCD a contiguous range of logical tiles so neighbours share its L2.
  const int total = gridDim.x;
  const int w = blockIdx.x;
  const int q = total >> 3, r = total & 7, x = w & 7;
  const int wl = x * q + (x < r ? x : r) + (w >> 3);
  const int per_batch = p.tiles_m * p.tiles_n;
  const int bidx = wl / per_batch;
  const int t = wl - bidx * per_batch;
  const int group = p.group_m * p.tiles_n;
  const int gid = t / group;
  const int first_m = gid * p.group_m;
  const int gm = min(p.tiles_m - first_m, p.group_m);
  const int within = t - gid * group;
  const int m0 = (first_m + within % gm) * BM;
  const int n0 = (within / gm) * BN;

  const int M = p.M, N = p.N, K = p.K;
  // 64-bit bases at the tile's origin (row m0 of A, column n0 of B), so only
  // offsets within one tile need 32 bits (the host checks BM*lda and
  // BK*ldb), whatever the size of the whole matrix.
  const int8_t *Ab = p.A + bidx * p.sa + (int64_t)m0 * p.lda;
  const int8_t *Bb = p.B + bidx * p.sb + (PACKED_B ? (int64_t)(n0 / 16) * p.ldb * 1024 : (int64_t)n0);

  // Per-thread global source offsets for one 64-deep k slice, relative to a
  // wave-uniform base that advances by one slice per step.
  uint32_t a_goff[CA];
  int a_lds[CA], a_k[CA];
#pragma unroll
  for (int i = 0; i < CA; ++i) {
    const int row = (tid >> 2) + 64 * i, c = tid & 3;
    int trow = row;
    if (EDGE) trow = min(m0 + row, M - 1) - m0;
    a_goff[i] = (uint32_t)((int64_t)trow * p.lda + c * 16);
    a_lds[i] = a_off(row, c);
    a_k[i] = c * 16;
  }
  int b_row[CB], b_lds[CB];
  uint32_t b_goff[CB];
#pragma unroll
  for (int i = 0; i < CB; ++i) {
    if constexpr (PACKED_B) {
      // chunk l of 1 KB tile t (16-column block n0/16 + t), kept in place
      const int ch = tid + 256 * i, t = ch >> 6, l = ch & 63;
      int tb = t;
      if (EDGE) tb = min(n0 / 16 + t, N / 16 - 1) - n0 / 16;
      b_row[i] = 0;
      b_goff[i] = (uint32_t)((int64_t)tb * p.ldb * 1024 + l * 16);
      b_lds[i] = t * 1024 + l * 16;
    } else {
      const int row = tid / BCH + (256 / BCH) * i, c = tid % BCH;
      int tcol = c * 16;
      if (EDGE) tcol = min(n0 + tcol, N - 16) - n0;
      b_row[i] = row;
      b_goff[i] = (uint32_t)((int64_t)row * p.ldb + tcol);
      b_lds[i] = row * BN + ((c ^ b_swz<BCH>(row)) << 4);
    }
  }

  const int KT = (K + BK - 1) / BK;
  // Global -> VGPR staging of k slice kt into (ra, rb). Slices past the last
  // one re-read the last slice (L2-resident); on the edge path their A part
  // is zero, so a padding step computes nothing, and elsewhere they are never
  // computed. The main loop thus has no data-dependent branches.
  auto load_slice = [&](int kt, v4i *ra, v4i *rb) {
    const int k0 = min(kt, KT - 1) * BK;
    const int8_t *abase = Ab + k0;
    const int8_t *bbase = Bb + (PACKED_B ? (int64_t)(k0 / BK) * 1024 : (int64_t)k0 * p.ldb);
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      if (EDGE == 2 && kt * BK + a_k[i] >= K) {
        ra[i] = v4i{0, 0, 0, 0};
      } else {
        ra[i] = *(const v4i *)(abase + a_goff[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      if (!PACKED_B && EDGE == 2 && k0 + b_row[i] >= K) {
        // rows past K: re-read row K-1 (A is zero there)
        rb[i] = *(const v4i *)(Bb + (int64_t)(K - 1 - b_row[i]) * p.ldb + b_goff[i]);
      } else {
        rb[i] = *(const v4i *)(bbase + b_goff[i]);
      }
    }
  };
  auto store_slice = [&](int buf, const v4i *ra, const v4i *rb) {
#pragma unroll
    for (int i = 0; i < CA; ++i) st_lds_b128(As0 + buf * A_BYTES, a_lds[i], ra[i]);
#pragma unroll
    for (int i = 0; i < CB; ++i) st_lds_b128(Bs0 + buf * B_BYTES, b_lds[i], rb[i]);
  };

  v16i acc[MI][NI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[mi][ni][e] = 0;

  // Fragment read offsets (within one slice buffer).
  const int g = lane >> 4, j = lane & 15;
  int a_frag[2][MI];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) {
      const int row = wm * WTM + mi * 32 + (lane & 31);
      a_frag[ks][mi] = a_off(row, ks * 2 + (lane >> 5));
    }
  int b_frag[2][NI];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) {
      if constexpr (PACKED_B) {
        const int t = (wn * WTN + ni * 32) / 16 + ((lane & 31) >> 4);
        b_frag[ks][ni] = t * 1024 + (16 * (2 * ks + (lane >> 5)) + (lane & 15)) * 16;
      } else {
        const int nc = (wn * WTN + ni * 32) / 16 + (g & 1);
        const int r0 = ks * 32 + (g >> 1) * 16 + (j >> 1);
        b_frag[ks][ni] = r0 * BN + ((nc ^ b_swz<BCH>(r0)) << 4) + (j & 1) * 8;
      }
    }

  // Fragments of one 32-deep k step: MI A blocks and NI B blocks.
  v4i fa0[MI], fb0[NI], fa1[MI], fb1[NI];
  auto read_frags = [&](int buf, int ks, v4i *fa, v4i *fb) {
    const int8_t *As = As0 + buf * A_BYTES;
    const int8_t *Bs = Bs0 + buf * B_BYTES;
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) fa[mi] = ld_lds_b128(As, a_frag[ks][mi]);
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) {
      if constexpr (PACKED_B) {
        fb[ni] = ld_lds_b128(Bs, b_frag[ks][ni]);
      } else {
        const v2i lo = ld_lds_tr8(Bs, b_frag[ks][ni]);
        const v2i hi = ld_lds_tr8(Bs, b_frag[ks][ni] + 8 * BN);
        fb[ni] = v4i{lo.x, lo.y, hi.x, hi.y};
      }
    }
  };
  auto mfma_block = [&](const v4i *fa, const v4i *fb) {
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
        acc[mi][ni] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[mi], fb[ni], acc[mi][ni], 0, 0, 0);
  };

  // Pipeline over three LDS buffers and two VGPR staging sets. Step kt
  // computes slice kt from buffer kt%3 while slice kt+2 goes VGPR -> LDS and
  // slice kt+4 goes global -> VGPR, so a global load has two steps to land.
  // Slice kt+1 was completed before the previous barrier, so its first
  // fragments are read before this step's barrier and the MFMA pipe does not
  // wait on LDS latency across steps. The single barrier per step also
  // guarantees every wave has finished reading buffer kt%3 before step kt+1
  // overwrites it with slice kt+3.
  // Small wave tiles (at most 4 accumulator blocks) hold the whole tile's
  // initial partial sums D in 64 registers, loaded in one round trip before
  // any C store (block-by-block loads would each wait for the previous
  // block's stores: vmcnt is in order). With EARLY_D they are loaded here,
  // so the round trip overlaps the k loop (~6 us less on a 128^3..512^3
  // GEMM), but 64 registers live across the loop cut occupancy from 3 waves
  // per SIMD to 1: the host asks for it only when the grid fits one
  // workgroup per CU. Otherwise they are loaded after the loop, when its
  // registers are free.
  constexpr bool D_TILE = HAS_D && MI * NI <= 4;
  constexpr bool D_EARLY = D_TILE && EARLY_D;
  int32_t d_pre[D_TILE ? MI : 1][D_TILE ? NI : 1][16];
  if constexpr (D_EARLY)
    load_d_tile<MI, NI, (EDGE > 0)>(d_pre, p.D + bidx * p.sd, p.ldd, m0 + wm * WTM, n0 + wn * WTN,
                                    M, N, lane);

  // SHORT (K <= 128, one pair of steps; the host picks it): slices 0 and 1
  // are both in flight before the first wait and nothing more is fetched,
  // so the k loop costs one global round trip instead of three. Longer K
  // keeps the general schedule below (the slices it fetches past the end
  // re-read the last one and are never computed).
  v4i ra0[CA], rb0[CB], ra1[CA], rb1[CB];
  if constexpr (SHORT) {
    load_slice(0, ra0, rb0);
    load_slice(1, ra1, rb1);
    store_slice(0, ra0, rb0);
    store_slice(1, ra1, rb1);
  } else {
    load_slice(0, ra0, rb0);
    store_slice(0, ra0, rb0);
    load_slice(1, ra1, rb1);
    store_slice(1, ra1, rb1);
    load_slice(2, ra0, rb0);
    load_slice(3, ra1, rb1);
  }
  lds_barrier();
  read_frags(0, 0, fa0, fb0);
  int b0 = 0, b1 = 1, b2 = 2;   // buffers of slices kt, kt+1, kt+2
  constexpr int NMFMA = MI * NI, NREAD = MI + (PACKED_B ? 1 : 2) * NI, NSTORE = CA + CB;
  auto step = [&](int kt, v4i *ra, v4i *rb) {
    // First half step: fragments of k 32..63 load under the MFMAs of k 0..31.
    read_frags(b0, 1, fa1, fb1);
    mfma_block(fa0, fb0);
#pragma unroll
    for (int i = 0; i < NMFMA; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                   // MFMA
      if (2 * i < NREAD) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read
    }
    __builtin_amdgcn_sched_barrier(0);
    // Second half step: slice kt+2 to LDS, slice kt+4 from memory (neither
    // exists with SHORT) and the next step's first fragments, interleaved
    // with the MFMAs of k 32..63.
    if constexpr (!SHORT) {
      store_slice(b2, ra, rb);
      load_slice(kt + 4, ra, rb);
    }
    read_frags(b1, 0, fa0, fb0);
    mfma_block(fa1, fb1);
#pragma unroll
    for (int i = 0; i < NMFMA; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);                   // MFMA
      if (i < NSTORE) {
        __builtin_amdgcn_sched_group_barrier(0x200, 1, 1);                 // DS write
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 1);                 // VMEM read
      } else if (2 * (i - NSTORE) < NREAD) {
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);                 // DS read
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
    const int bt = b0;
    b0 = b1;
    b1 = b2;
    b2 = bt;
  };
  // Two steps per iteration (one per staging set). An odd step count only
  // occurs with EDGE == 2 (the host routes K % 128 != 0 there), where the
  // padding step multiplies zero A columns.
  if constexpr (SHORT) {
    step(0, ra0, rb0);
    step(1, ra1, rb1);
  } else {
    for (int kt = 0; kt < KT; kt += 2) {
      step(kt, ra0, rb0);
      step(kt + 1, ra1, rb1);
    }
  }

  if constexpr (D_TILE) {
    if constexpr (!D_EARLY)
      load_d_tile<MI, NI, (EDGE > 0)>(d_pre, p.D + bidx * p.sd, p.ldd, m0 + wm * WTM, n0 + wn * WTN,
                                      M, N, lane);
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[mi][ni][e] = add_wrap(acc[mi][ni][e], d_pre[mi][ni][e]);
    store_tile<MI, NI, (EDGE > 0), false>(acc, p.C + bidx * p.sc, nullptr, p.ldc, p.ldd,
                                    m0 + wm * WTM, n0 + wn * WTN, M, N, lane);
  } else {
    store_tile<MI, NI, (EDGE > 0), HAS_D>(acc, p.C + bidx * p.sc, HAS_D ? p.D + bidx * p.sd : nullptr,
                                    p.ldc, p.ldd, m0 + wm * WTM, n0 + wn * WTN, M, N, lane);
  }
}

// ---------------------------------------------------------------------------
// Full-tile MFMA kernel with direct-to-LDS loads (256 x 256 tiles)
// ---------------------------------------------------------------------------

// Static LDS per workgroup of the persistent 256x256 kernels (one workgroup
// per CU): gemm_dma_kernel's 4 slice stages, and gemm_dma16_kernel's 4 stages
// plus the 8 KB epilogue strip of each of its 4 waves.
constexpr int kDmaLds = 4 * (256 * 64 + 64 * 256);
constexpr int kDma16Lds = kDmaLds + 4 * 8192;

// gfx950 LDS DMA: each lane of the wave fetches the 16 global bytes at
// base + voff and the wave writes them, in lane order, to the 1 KB of LDS
// starting at m0. The LDS stores are tracked by vmcnt like any global load;
// the caller waits with s_waitcnt vmcnt before a barrier publishes them.
__device__ __forceinline__ void dma_b128(const int8_t *base, uint32_t voff, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(base), "s"(m0));
}

// Same contract as gemm_mfma_kernel<256, 256, EDGE, HAS_D, false> for
// M, N >= 256 and K % 64 == 0 (a last tile row or column that would pass M or
// N starts at M - 256 or N - 256 instead, so no load or store leaves A, B, C
// or D), but the k slices go global -> LDS
// by DMA (no VGPR staging, no ds_write instructions) and the kernel is
// persistent: one workgroup per CU walks its tiles in order and the slice
// stream runs on across tile boundaries, so the last steps of a tile already
// fetch the first slices of the next one and a tile change costs only its
// C stores.
//
// Slices are numbered globally, g = (tile iteration) * KT + kt. Four LDS
// stages: step g computes slice g from stage g%4, reads the first fragments of
// slice g+1 early, and issues the DMA of slice g+3 into stage (g+3)%4 (last
// read in step g-1). The wait at the end of step g (vmcnt(8): only slice
// g+3's eight DMAs per wave may still be in flight) plus the barrier publish
// slice g+2 before step g+1 reads its fragments early.
//
// WAVES = 4: one wave per SIMD, each owning a 128x128 block (2x2 layout).
// WAVES = 8: two waves per SIMD, each owning a 128x64 block (2 rows x 4
// columns of waves), so while one wave of a SIMD waits (a DMA the memory
// pipeline cannot take yet, a C store burst) the other keeps its MFMA pipe
// busy; fragment reads per MFMA rise by a third.
//
// PACKED_B: B is in the packed layout of vt_pack_b_i8 (p.B = Bp, p.ldb = kbt,
// the 64-row blocks per 16-column block, p.sb = the packed batch stride). A
// slice's B is then 16 whole 1 KB tiles, one per 16-column block, each a
// single DMA of contiguous bytes, and each tile holds lane l's 16 consecutive
// k of column l % 16 at byte 16 * l. A lane's B operand of the 32x32x32 MFMA
// (column l % 32, k 16 * (l / 32) .. +15 of the 32-deep step, the same k as
// its A operand) is one ds_read_b128: two fragment reads per B block fewer
// than the transposing ds_read_b64_tr_b8 pair that row-major B needs.
// EDGE: M or N is not a whole number of tiles; a last tile row or column
// starts at M - 256 or N - 256, and the rows and columns it shares with its
// neighbour are left to the neighbour's stores.
template <int WAVES, bool HAS_D, bool PACKED_B = false, bool EDGE = false>
__global__ __launch_bounds__(64 * WAVES, 1) void gemm_dma_kernel(GemmArgs p) {
  static_assert(WAVES == 4 || WAVES == 8, "4 or 8 waves");
  constexpr int BM = 256, BN = 256, BK = 64;
  constexpr int WTM = 128, WTN = WAVES == 4 ? 128 : 64, MI = WTM / 32, NI = WTN / 32;
  constexpr int BCH = BN / 16;
  constexpr int A_BYTES = BM * BK, B_BYTES = BK * BN, STAGE = A_BYTES + B_BYTES;
  constexpr int NSTAGE = 4;
  constexpr int DPW = 16 / WAVES;        // 1 KB DMA blocks of A (and of B) per wave per slice
  constexpr int DMAS = 2 * DPW;          // DMAs per wave per slice
  __shared__ __attribute__((aligned(1024))) int8_t smem[NSTAGE * STAGE];
  static_assert(sizeof(smem) == kDmaLds, "LDS the host reports for this kernel");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = WAVES == 4 ? wave >> 1 : wave & 1;
  const int wn = WAVES == 4 ? wave & 1 : wave >> 1;

  // This workgroup computes logical tiles wl, wl + G, wl + 2G, ... where wl
  // is its XCD-contiguous rank (workgroup w runs on XCD w % 8), so the tiles
  // in flight on one XCD form a compact block that shares its L2.
  const int G = gridDim.x;
  const int w = blockIdx.x;
  const int q = G >> 3, r = G & 7, x = w & 7;
  const int wl = x * q + (x < r ? x : r) + (w >> 3);
  const int per_batch = p.tiles_m * p.tiles_n;
  const int total_tiles = per_batch * p.batch_count;
  if (wl >= total_tiles) return;
  const int ntiles = (total_tiles - 1 - wl) / G + 1;
  const int group = p.group_m * p.tiles_n;
  // Tile iteration -> (batch, row origin, column origin, and the origins
  // before a last tile row or column is moved back).
  auto tile_coords = [&](int it, int &bidx, int &m0, int &n0, int &mn, int &nn) {
    const int lt = wl + it * G;
    bidx = lt / per_batch;
    const int t = lt - bidx * per_batch;
    const int gid = t / group;
    const int first_m = gid * p.group_m;
    const int gm = min(p.tiles_m - first_m, p.group_m);
    const int within = t - gid * group;
    // A last tile row or column past M or N is moved back to end at M or N
    // (the launch ensures M, N >= 256). It recomputes rows or columns of its
    // neighbour and does not store them (store_tile's lower bounds).
    mn = (first_m + within % gm) * BM;
    nn = (within / gm) * BN;
    m0 = min(mn, p.M - BM);
    n0 = min(nn, p.N - BN);
  };

  const int64_t lda = p.lda, ldb = p.ldb;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(LDS_AS int8_t *)smem;
  const int KT = p.K / BK;
  const int last_g = ntiles * KT - 1;

  // DMA sources. Wave w fills A blocks DPW*w .. DPW*w+DPW-1 (16 rows of 64
  // bytes each) and the same B blocks (4 rows of 256 bytes each; with packed
  // B, the 1 KB tiles of 16-column blocks DPW*w ..); lane L lands at byte
  // 16*L of its block, so it fetches the logical chunk that the swizzle maps
  // to that position (XOR swizzles are their own inverse). Lane offsets are
  // relative to the tile's origin, which goes into the wave-uniform base.
  uint32_t a_lane[DPW], b_lane[DPW];
#pragma unroll
  for (int i = 0; i < DPW; ++i) {
    const int arow = (wave * DPW + i) * 16 + (lane >> 2);
    const int ac = (lane & 3) ^ a_swz(arow);
    a_lane[i] = (uint32_t)((int64_t)arow * lda + ac * 16);
    if constexpr (PACKED_B) {
      b_lane[i] = (uint32_t)((int64_t)(wave * DPW + i) * ldb * 1024 + lane * 16);
    } else {
      const int brow = (wave * DPW + i) * 4 + (lane >> 4);
      const int bc = (lane & 15) ^ b_swz<BCH>(brow);
      b_lane[i] = (uint32_t)((int64_t)brow * ldb + bc * 16);
    }
  }
  // The slice the next DMA fetches, as (tile iteration, k slice), advanced one
  // slice per DMA round; tile origins are recomputed only at tile changes.
  // Slices past the last one re-read it (their stages are never read).
  int d_it = 0, d_kt = 0;
  const int8_t *a_tile = nullptr, *b_tile = nullptr;
  auto set_tile = [&](int it) {
    int bidx, m0, n0, mn, nn;
    tile_coords(it, bidx, m0, n0, mn, nn);
    a_tile = p.A + bidx * p.sa + (int64_t)m0 * lda;
    b_tile = p.B + bidx * p.sb + (PACKED_B ? (int64_t)(n0 / 16) * ldb * 1024 : (int64_t)n0);
  };
  set_tile(0);
  auto next_bases = [&](const int8_t *&abase, const int8_t *&bbase) {
    abase = a_tile + d_kt * BK;
    bbase = b_tile + (PACKED_B ? (int64_t)d_kt * 1024 : (int64_t)(d_kt * BK) * ldb);
    if (d_it * KT + d_kt < last_g) {
      if (++d_kt == KT) {
        d_kt = 0;
        set_tile(++d_it);
      }
    }
  };
  auto issue_slice = [&](int stage) {
    const int8_t *abase, *bbase;
    next_bases(abase, bbase);
    const uint32_t ma = lds0 + stage * STAGE + wave * DPW * 1024;
    const uint32_t mb = ma + A_BYTES;
#pragma unroll
    for (int i = 0; i < DPW; ++i) dma_b128(abase, a_lane[i], ma + i * 1024);
#pragma unroll
    for (int i = 0; i < DPW; ++i) dma_b128(bbase, b_lane[i], mb + i * 1024);
  };

  const int g = lane >> 4, j = lane & 15;
  int a_frag[2][MI], b_frag[2][NI];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
      a_frag[ks][mi] = a_off(wm * WTM + mi * 32 + (lane & 31), ks * 2 + (lane >> 5));
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) {
      if constexpr (PACKED_B) {
        const int t = (wn * WTN + ni * 32) / 16 + ((lane & 31) >> 4);
        b_frag[ks][ni] = t * 1024 + (16 * (2 * ks + (lane >> 5)) + (lane & 15)) * 16;
      } else {
        const int nc = (wn * WTN + ni * 32) / 16 + (g & 1);
        const int r0 = ks * 32 + (g >> 1) * 16 + (j >> 1);
        b_frag[ks][ni] = r0 * BN + ((nc ^ b_swz<BCH>(r0)) << 4) + (j & 1) * 8;
      }
    }
  }
  v16i acc[MI][NI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[mi][ni][e] = 0;

  // Fragments of one 32-deep k step as MI + BU LDS reads ("units"): units
  // 0..MI-1 are the A blocks (ds_read_b128), the rest the lo/hi halves of the
  // B blocks (ds_read_b64_tr_b8), or with packed B the whole B blocks
  // (ds_read_b128).
  constexpr int BU = PACKED_B ? NI : 2 * NI;
  constexpr int NUNIT = MI + BU;
  static_assert(NUNIT <= 15, "the barrier's lgkmcnt counts one k step of reads");
  v4i fa0[MI], fa1[MI];
  v2i fl0[NI], fh0[NI], fl1[NI], fh1[NI];   // row-major B
  v4i fb0[NI], fb1[NI];                     // packed B
  auto read_unit = [&](int stage, int ks, int u, v4i *fa, v2i *fl, v2i *fh, v4i *fb) {
    const int8_t *As = smem + stage * STAGE;
    const int8_t *Bs = As + A_BYTES;
    if (u < MI) {
      fa[u] = ld_lds_b128(As, a_frag[ks][u]);
    } else if constexpr (PACKED_B) {
      fb[u - MI] = ld_lds_b128(Bs, b_frag[ks][u - MI]);
    } else {
      const int ni = (u - MI) >> 1;
      if (((u - MI) & 1) == 0) fl[ni] = ld_lds_tr8(Bs, b_frag[ks][ni]);
      else fh[ni] = ld_lds_tr8(Bs, b_frag[ks][ni] + 8 * BN);
    }
  };
  auto mfma = [&](int mi, int ni, const v4i *fa, const v2i *fl, const v2i *fh, const v4i *fb) {
    const v4i b = PACKED_B ? fb[ni] : v4i{fl[ni].x, fl[ni].y, fh[ni].x, fh[ni].y};
    acc[mi][ni] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[mi], b, acc[mi][ni], 0, 0, 0);
  };

  issue_slice(0);
  issue_slice(1);
  issue_slice(2);
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" :: "n"(DMAS) : "memory");   // slices 0, 1 landed
#pragma unroll
  for (int u = 0; u < NUNIT; ++u) read_unit(0, 0, u, fa0, fl0, fh0, fb0);

  int gs = 0;   // global slice index
  for (int it = 0; it < ntiles; ++it) {
    // Once per tile: wait for every LDS read and scalar load. The compiler
    // hoists epilogue kernel-argument loads (s_load) above the tile loop, and
    // scalar loads retire out of order with LDS reads; left pending into the
    // k loop they make every step open with lgkmcnt(0), a full LDS round trip
    // on the first MFMA of each 64-deep slice. Cleared here, the steps keep
    // their early fragment reads in flight across the barrier.
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0); vmcnt, expcnt untouched
    // Explicit schedule over the 32 MFMA slots of a slice, one MFMA per
    // scheduling region: slots 0-15 multiply the k 0..31 fragments of slice
    // gs while the k 32..63 fragments of slice gs are read (one per slot, in
    // the order the next slots need them); slots 16-31 multiply those while
    // the k 0..31 fragments of slice gs+1 (published by the previous barrier)
    // are read. The DMAs of slice gs+3 go out one every four slots so the
    // memory pipeline sees a steady stream instead of a burst.
    for (int kt = 0; kt < KT; ++kt, ++gs) {
      const int s0 = gs & 3, s1 = (gs + 1) & 3, s3 = (gs + 3) & 3;
      const int8_t *abase, *bbase;
      next_bases(abase, bbase);   // slice gs+3
      const uint32_t ma = lds0 + s3 * STAGE + wave * DPW * 1024;
      const uint32_t mb = ma + A_BYTES;
      // Read order = first use: A0 and the B blocks (MFMAs 0..NI-1), then A1..
#pragma unroll
      for (int slot = 0; slot < 2 * MI * NI; ++slot) {
        const int i = slot % (MI * NI);
        const int u = i == 0 ? 0 : i <= BU ? MI + i - 1 : i - BU;
        if (slot < MI * NI) {
          mfma(i / NI, i % NI, fa0, fl0, fh0, fb0);
          if (i < NUNIT) read_unit(s0, 1, u, fa1, fl1, fh1, fb1);
        } else {
          mfma(i / NI, i % NI, fa1, fl1, fh1, fb1);
          if (i < NUNIT) read_unit(s1, 0, u, fa0, fl0, fh0, fb0);
        }
        if ((slot & 3) == 2) {
          const int d = slot >> 2;
          if (d < DPW) dma_b128(abase, a_lane[d], ma + d * 1024);
          else dma_b128(bbase, b_lane[d - DPW], mb + (d - DPW) * 1024);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      // Slice gs+2 has landed (only slice gs+3's DMAs remain in flight; older
      // stores are waited for as well) and every read of stage s0 has
      // completed (only the NUNIT reads of stage s1 remain), so after the
      // barrier step gs+1 may refill stage s0.
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(%1)\n\ts_barrier" :: "n"(DMAS), "n"(NUNIT) : "memory");
    }
    int bidx, m0, n0, mn, nn;
    tile_coords(it, bidx, m0, n0, mn, nn);
    store_tile<MI, NI, false, HAS_D, EDGE>(acc, p.C + bidx * p.sc,
                                           HAS_D ? p.D + bidx * p.sd : nullptr, p.ldc, p.ldd,
                                           m0 + wm * WTM, n0 + wn * WTN, p.M, p.N, lane, mn, nn);
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[mi][ni][e] = 0;
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// ---------------------------------------------------------------------------
// Full-tile MFMA kernel on v_mfma_i32_16x16x64_i8
// ---------------------------------------------------------------------------

// Slice swizzles of gemm_dma16_kernel. A slice [256][64 B]: a 16x16x64 A
// fragment read (lane l: row l % 16, chunk l / 16) puts rows r and r + 8 in one
// ds_read_b128 lane group, so chunk c of row r is stored at c ^ (2 * bit 3 of
// r). B slice [64][256 B]: the transposing reads of one 32-lane group take
// rows r .. r + 7 and r + 16 .. r + 23 of one chunk, so chunk c of row r is
// stored at c ^ (r % 8 + 8 * bit 4 of r). Both give every lane group distinct
// banks under the measured grouping (helpers above).
__device__ __forceinline__ int a16_swz(int row) { return ((row >> 3) & 1) << 1; }
__device__ __forceinline__ int a16_off(int row, int c) { return row * 64 + ((c ^ a16_swz(row)) << 4); }
__device__ __forceinline__ int b16_swz(int row) { return (row & 7) | (((row >> 4) & 1) << 3); }
// B slice [64][128 B] of the 256x128 form: the 16 rows of one 32-lane
// transposing read (r .. r + 7 and r + 16 .. r + 23) fall on two bank halves
// by row parity, so the 8 rows of each parity need 8 distinct chunks: chunk c
// of row r is stored at c ^ ((r / 2) % 4 + 4 * bit 4 of r).
__host__ __device__ constexpr int b8_swz(int row) { return ((row >> 1) & 3) | (((row >> 4) & 1) << 2); }

// Epilogue of gemm_dma16_kernel through LDS: each 16-row strip of the wave's
// 128-column block is written to the wave's 8 KB of LDS in the accumulator
// layout and read back row-contiguous, so every global store is 16 bytes per
// lane and one instruction writes two whole 512-byte row segments (the
// accumulator layout gives 64-byte row segments). 16-byte chunk k of strip
// row r is stored at chunk k ^ (4 * ((r / 4) % 4)): the 4-byte writes of one
// instruction (rows 4 * (l / 16) + e, column l % 16 of a block) then fall on
// 64 distinct banks, and each 16-lane read still covers 16 distinct chunks of
// one row. With D, the strip's D values (the same row-contiguous 16 bytes each
// lane then stores) are all loaded before its stores; each lane reads its own
// D bytes before writing them, so C may be D.
__host__ __device__ constexpr int strip_off(int row, int chunk) {
  return row * 512 + ((chunk ^ (((row >> 2) & 3) << 2)) << 4);
}

// Per-lane addressing of the epilogue strip, computed once per kernel so
// that every strip access is a base register plus an immediate offset.
// Write of element e of block ni (strip row 4 g + e, g = lane / 16, column
// 16 ni + lane % 16): wb[ni % 4] + 512 e + 64 (ni & 4). Read j (strip row
// 2 j + lane / 32, chunk lane % 32): rb[j / 2] + 1024 j. The bases include
// the strip's own offset in LDS. gofs_c / gofs_d: byte offset of the lane's
// 16 bytes from the start of its row pair (row 2 j of the strip, the wave's
// first column).
__host__ __device__ constexpr int strip_wb(int lane, int k) {
  return 2048 * (lane >> 4) + (((k ^ (lane >> 4)) & 3) << 6) + (lane & 15) * 4;
}
__host__ __device__ constexpr int strip_rb(int lane, int m) {
  return 512 * (lane >> 5) + (((lane & 31) ^ (m << 2)) << 4);
}

// The bases give strip_off's layout for every lane, block, element and read.
constexpr bool strip_bases_match() {
  for (int lane = 0; lane < 64; ++lane) {
    const int g = lane >> 4, c = lane & 15;
    for (int ni = 0; ni < 8; ++ni)
      for (int e = 0; e < 4; ++e)
        if (strip_wb(lane, ni & 3) + 512 * e + 64 * (ni & 4) !=
            strip_off(4 * g + e, ni * 4 + (c >> 2)) + (c & 3) * 4)
          return false;
    for (int j = 0; j < 8; ++j)
      if (strip_rb(lane, j >> 1) + 1024 * j != strip_off(2 * j + (lane >> 5), lane & 31)) return false;
  }
  return true;
}
static_assert(strip_bases_match(), "strip bases disagree with strip_off");

// The 64-column strip of the 256x128 form: 16 rows of 256 bytes, chunk k of
// row r at k ^ (4 * ((r / 4) % 4)). Write of element e of block ni (row
// 4 g + e, column 16 ni + c, g = lane / 16, c = lane % 16): wb[ni] + 256 e.
// Read j (row 4 j + lane / 16, chunk lane % 16): rb[j] + 1024 j.
__host__ __device__ constexpr int strip64_off(int row, int chunk) {
  return row * 256 + ((chunk ^ (((row >> 2) & 3) << 2)) << 4);
}
__host__ __device__ constexpr int strip64_wb(int lane, int ni) {
  return 1024 * (lane >> 4) + 64 * (ni ^ (lane >> 4)) + 4 * (lane & 15);
}
__host__ __device__ constexpr int strip64_rb(int lane, int j) {
  return 256 * (lane >> 4) + (((lane & 15) ^ (4 * j)) << 4);
}
constexpr bool strip64_bases_match() {
  for (int lane = 0; lane < 64; ++lane) {
    const int g = lane >> 4, c = lane & 15;
    for (int ni = 0; ni < 4; ++ni)
      for (int e = 0; e < 4; ++e)
        if (strip64_wb(lane, ni) + 256 * e != strip64_off(4 * g + e, 4 * ni + (c >> 2)) + (c & 3) * 4)
          return false;
    for (int j = 0; j < 4; ++j)
      if (strip64_rb(lane, j) + 1024 * j != strip64_off(4 * j + g, c)) return false;
  }
  return true;
}
static_assert(strip64_bases_match(), "64-column strip bases disagree with strip64_off");

struct StripLanes {
  int wb[4], rb[4];
  uint32_t gofs_c, gofs_d;
};

__device__ __forceinline__ StripLanes strip_lanes(int lane, int strip_base, int64_t ldc, int64_t ldd) {
  StripLanes s;
#pragma unroll
  for (int k = 0; k < 4; ++k) s.wb[k] = strip_base + strip_wb(lane, k);
#pragma unroll
  for (int m = 0; m < 4; ++m) s.rb[m] = strip_base + strip_rb(lane, m);
  s.gofs_c = (uint32_t)(((lane >> 5) * ldc + (lane & 31) * 4) * 4);
  s.gofs_d = (uint32_t)(((lane >> 5) * ldd + (lane & 31) * 4) * 4);
  return s;
}

// One 16-row strip of store_tile16_lds: Cs / Ds point at the strip's first
// row and the wave's first column. MASKED: store j of a lane writes only when
// row_rel + 2 j >= 0 and col_ok (a moved-back tile leaves the rows and
// columns it shares with its neighbour to the neighbour).
template <int NI, bool HAS_D, bool MASKED = false>
__device__ __forceinline__ void store_strip16_lds(const v4i (&acc)[NI], int32_t *Cs,
                                                  const int32_t *Ds, int64_t ldc, int64_t ldd,
                                                  const StripLanes &sl, LDS_AS int8_t *lds,
                                                  int row_rel = 0, bool col_ok = true) {
  static_assert(NI * 16 == 128, "two 512-byte rows per wave instruction");
#pragma unroll
  for (int ni = 0; ni < NI; ++ni)
#pragma unroll
    for (int e = 0; e < 4; ++e)
      *(LDS_AS int32_t *)(lds + sl.wb[ni & 3] + e * 512 + (ni & 4) * 64) = acc[ni][e];
  v4i v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = *(LDS_AS v4i *)(lds + sl.rb[j >> 1] + j * 1024);
  if constexpr (HAS_D) {
    v4i d[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      d[j] = *(const v4i *)((const int8_t *)(Ds + 2 * j * ldd) + sl.gofs_d);
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) v[j][q] = add_wrap(v[j][q], d[j][q]);
    // Masked: the sums are formed before the conditional stores. Sunk into
    // them, a masked lane's D load would stay outstanding into the next
    // tile, where the compiler waits for all vector memory (vmcnt(0))
    // before reusing its register in the k loop.
    if constexpr (MASKED) {
#pragma unroll
      for (int j = 0; j < 8; ++j) asm volatile("" : "+v"(v[j]));
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (!MASKED || (col_ok && row_rel + 2 * j >= 0))
      __builtin_nontemporal_store(v[j], (v4i *)((int8_t *)(Cs + 2 * j * ldc) + sl.gofs_c));
}

// row_rel0: the lane's row in the wave's first strip (2 j + lane / 32 for
// store j) less the rows the tile leaves to its neighbour (MASKED).
template <int MI, int NI, bool HAS_D, int FIRST = 0, bool MASKED = false>
__device__ __forceinline__ void store_tile16_lds(const v4i (&acc)[MI][NI], int32_t *Cb,
                                                 const int32_t *Db, int64_t ldc, int64_t ldd,
                                                 const StripLanes &sl, LDS_AS int8_t *lds,
                                                 int row_rel0 = 0, bool col_ok = true) {
#pragma unroll
  for (int mi = FIRST; mi < MI; ++mi) {
    store_strip16_lds<NI, HAS_D, MASKED>(acc[mi], Cb + mi * 16 * ldc,
                                         HAS_D ? Db + mi * 16 * ldd : nullptr, ldc, ldd, sl, lds,
                                         row_rel0 + mi * 16, col_ok);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// One 16-row strip of the 256x128 form's epilogue: the wave's 64 columns go
// through its LDS strip and out as 4 stores, each of four whole 256-byte row
// segments. wb / rb: strip64_wb / strip64_rb plus the strip's offset in LDS;
// gofs_c / gofs_d: the lane's byte offset from its 4-row group's base. With
// D, the strip's 4 D loads precede its stores, and each lane reads its own D
// bytes before writing them, so C may be D. MASKED: store j of a lane writes
// only when row_rel + 4 j >= 0 and col_ok (a moved-back tile leaves the rows
// and columns it shares with its neighbour to the neighbour).
template <bool HAS_D, bool MASKED = false>
__device__ __forceinline__ void store_strip64_lds(const v4i (&acc)[4], int32_t *Cs, const int32_t *Ds,
                                                  int64_t ldc, int64_t ldd, const int (&wb)[4],
                                                  const int (&rb)[4], uint32_t gofs_c, uint32_t gofs_d,
                                                  LDS_AS int8_t *lds, int row_rel = 0,
                                                  bool col_ok = true) {
#pragma unroll
  for (int ni = 0; ni < 4; ++ni)
#pragma unroll
    for (int e = 0; e < 4; ++e) *(LDS_AS int32_t *)(lds + wb[ni] + e * 256) = acc[ni][e];
  v4i v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = *(LDS_AS v4i *)(lds + rb[j] + j * 1024);
  if constexpr (HAS_D) {
    v4i d[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) d[j] = *(const v4i *)((const int8_t *)(Ds + 4 * j * ldd) + gofs_d);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) v[j][q] = add_wrap(v[j][q], d[j][q]);
    // Masked: the sums are formed before the conditional stores (as in
    // store_strip16_lds), so no masked lane's D load stays outstanding.
    if constexpr (MASKED) {
#pragma unroll
      for (int j = 0; j < 4; ++j) asm volatile("" : "+v"(v[j]));
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (!MASKED || (col_ok && row_rel + 4 * j >= 0))
      __builtin_nontemporal_store(v[j], (v4i *)((int8_t *)(Cs + 4 * j * ldc) + gofs_c));
}

// v_mfma_i32_16x16x64_i8 accumulating in place in AGPRs. As a builtin, the
// compiler gives each result a new register tuple and, with all 256 AGPRs
// holding accumulators, stages them through VGPRs around every MFMA; the
// tied asm operand keeps each accumulator in one AGPR tuple. Hazards: every
// use in gemm_dma16_kernel reads an accumulator 32 or 64 MFMAs after its previous
// write, its fragments come from LDS reads the compiler waits for, and the
// kernel waits explicitly before its epilogue reads the results.
__device__ __forceinline__ void mfma16_in_place(v4i &acc, const v4i &a, const v4i &b) {
  asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

// Same contract and structure as gemm_dma_kernel<4, HAS_D, PACKED_B, EDGE>
// (256x256 tiles, the last ones moved back to end at M and N when EDGE,
// persistent, k slices by DMA into 4 LDS stages, 3 slices ahead, one barrier
// per slice), with each wave's 128x128 block held as 8 x 8
// v_mfma_i32_16x16x64_i8 accumulators instead of 4 x 4 of 32x32x32. The
// 16x16x64 form does the same work per slice from the same 16 KB of fragment
// reads per wave, and on config-5 data its register-only loop sustains about
// 20 % more operations per second at the board's power limit (3945 against
// 3262-3293 TOPS, at 1.98 against 1.67 GHz): it reads and writes half the
// accumulator bytes per multiply-add.
//
// Step gs multiplies slice gs (its whole 64-deep fragment set, read during
// step gs - 1) in 64 MFMA slots while reading slice gs + 1's fragments into
// the other register set, one LDS read per slot in first-use order, and
// issues slice gs + 3's DMAs one every 8 slots. The wait at the end of step gs
// (vmcnt(DMAS): only slice gs + 3's DMAs may remain) plus the barrier publish
// slice gs + 2, whose fragments step gs + 1 reads. Stage gs % 4 is refilled in
// step gs + 1; its reads were issued in step gs - 1 and consumed by step gs's
// MFMAs. The 256x128 form (BN = 128) runs the same schedule over 32 slots,
// with 6 DMAs per slice issued one every 4 slots.
template <bool HAS_D, bool PACKED_B, bool EDGE = false, int BN = 256>
__global__ __launch_bounds__(256, 1) void gemm_dma16_kernel(GemmArgs p) {
  // BN = 128 (the 256x128 form) gives each wave a 128x64 block and half the
  // B slice; the rest is shared.
  static_assert(BN == 256 || BN == 128, "256x256 or 256x128 tiles");
  constexpr int BM = 256, BK = 64;
  constexpr int WTM = 128, WTN = BN / 2, MI = WTM / 16, NI = WTN / 16;
  constexpr int A_BYTES = BM * BK, B_BYTES = BK * BN;
  constexpr int NSTAGE = 4;
  // A stages at [0, 64 KB), B stages at [64 KB, 128 KB) (each B stage in a
  // 16 KB slot): with the stage a compile-time constant, every fragment read
  // is its base register plus an immediate offset below 64 KB, with no
  // address arithmetic per read.
  constexpr int B_REGION = NSTAGE * A_BYTES;
  static_assert(B_BYTES <= A_BYTES && (NSTAGE - 1) * A_BYTES + 8 * BN < 65536, "16-bit read offsets");
  constexpr int DPW = 4;                 // 1 KB DMA blocks of A per wave per slice
  constexpr int DPW_B = B_BYTES / 4096;  // and of B (4 or 2)
  constexpr int DMAS = DPW + DPW_B;
  // The 32 KB past the stages hold each wave's 8 KB epilogue strip.
  __shared__ __attribute__((aligned(1024))) int8_t smem[NSTAGE * 2 * A_BYTES + 4 * 8192];
  static_assert(sizeof(smem) == kDma16Lds, "LDS the host reports for this kernel");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  const int G = gridDim.x;
  const int w = blockIdx.x;
  const int q = G >> 3, r = G & 7, x = w & 7;
  const int wl = x * q + (x < r ? x : r) + (w >> 3);
  const int per_batch = p.tiles_m * p.tiles_n;
  const int total_tiles = per_batch * p.batch_count;
  if (wl >= total_tiles) return;
  const int ntiles = (total_tiles - 1 - wl) / G + 1;
  const int group = p.group_m * p.tiles_n;
  auto tile_coords = [&](int it, int &bidx, int &m0, int &n0, int &mn, int &nn) {
    const int lt = wl + it * G;
    bidx = lt / per_batch;
    const int t = lt - bidx * per_batch;
    const int gid = t / group;
    const int first_m = gid * p.group_m;
    const int gm = min(p.tiles_m - first_m, p.group_m);
    const int within = t - gid * group;
    mn = (first_m + within % gm) * BM;   // last tiles end at M, N
    nn = (within / gm) * BN;
    m0 = min(mn, p.M - BM);
    n0 = min(nn, p.N - BN);
  };

  const int64_t lda = p.lda, ldb = p.ldb;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(LDS_AS int8_t *)smem;
  const int KT = p.K / BK;
  const int last_g = ntiles * KT - 1;

  uint32_t a_lane[DPW], b_lane[DPW];
#pragma unroll
  for (int i = 0; i < DPW; ++i) {
    const int arow = (wave * DPW + i) * 16 + (lane >> 2);
    const int ac = (lane & 3) ^ a16_swz(arow);
    a_lane[i] = (uint32_t)((int64_t)arow * lda + ac * 16);
    if constexpr (PACKED_B) {
      // whole 1 KB tiles of column blocks wave * DPW_B + i
      b_lane[i] = i < DPW_B ? (uint32_t)((int64_t)(wave * DPW_B + i) * ldb * 1024 + lane * 16) : 0;
    } else if constexpr (BN == 256) {
      const int brow = (wave * DPW + i) * 4 + (lane >> 4);
      const int bc = (lane & 15) ^ b16_swz(brow);
      b_lane[i] = (uint32_t)((int64_t)brow * ldb + bc * 16);
    } else if (i < DPW_B) {
      // 8 rows of 128 bytes per 1 KB block; lane L writes slot L % 8 of row L / 8
      const int brow = (wave * DPW_B + i) * 8 + (lane >> 3);
      const int bc = (lane & 7) ^ b8_swz(brow);
      b_lane[i] = (uint32_t)((int64_t)brow * ldb + bc * 16);
    } else {
      b_lane[i] = 0;
    }
  }
  // The slice the next DMA round fetches: running A and B pointers, the
  // slices left in the current tile and in the whole walk (slices past the
  // last one re-read it; their stages are never read).
  int d_it = 0, d_left = KT, g_left = last_g;
  const int8_t *a_next = nullptr, *b_next = nullptr;
  const int64_t b_step = PACKED_B ? 1024 : (int64_t)BK * ldb;
  auto set_tile = [&](int it) {
    int bidx, m0, n0, mn, nn;
    tile_coords(it, bidx, m0, n0, mn, nn);
    a_next = p.A + bidx * p.sa + (int64_t)m0 * lda;
    b_next = p.B + bidx * p.sb + (PACKED_B ? (int64_t)(n0 / 16) * ldb * 1024 : (int64_t)n0);
  };
  set_tile(0);
  auto next_bases = [&](const int8_t *&abase, const int8_t *&bbase) {
    abase = a_next;
    bbase = b_next;
    if (g_left > 0) {
      --g_left;
      if (--d_left == 0) {
        d_left = KT;
        set_tile(++d_it);
      } else {
        a_next += BK;
        b_next += b_step;
      }
    }
  };
  auto issue_slice = [&](int stage) {
    const int8_t *abase, *bbase;
    next_bases(abase, bbase);
    const uint32_t ma = lds0 + stage * A_BYTES + wave * DPW * 1024;
    const uint32_t mb = BN == 256 ? ma + B_REGION : lds0 + B_REGION + stage * A_BYTES + wave * DPW_B * 1024;
#pragma unroll
    for (int i = 0; i < DPW; ++i) dma_b128(abase, a_lane[i], ma + i * 1024);
#pragma unroll
    for (int i = 0; i < DPW_B; ++i) dma_b128(bbase, b_lane[i], mb + i * 1024);
  };

  // Fragment offsets within a stage. A block mi: lane l reads row
  // wm*128 + mi*16 + l%16, chunk l/16 (k 16*(l/16) .. +15). B block ni (columns
  // wn*128 + ni*16 ..): lane l needs k 16*(l/16) .. +15 of column l%16, read as
  // two transposed 8-row halves (rows 16*(l/16) + (l%16)/2 and + 8, the same
  // swizzle), or with packed B as one 16-byte piece of the block's tile.
  int a_frag[MI], b_frag[NI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi) a_frag[mi] = a16_off(wm * WTM + mi * 16 + (lane & 15), lane >> 4);
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    const int cb = wn * (WTN / 16) + ni;
    if constexpr (PACKED_B) {
      b_frag[ni] = B_REGION + cb * 1024 + lane * 16;
    } else {
      const int row = 16 * (lane >> 4) + ((lane & 15) >> 1);
      const int swz = BN == 256 ? b16_swz(row) : b8_swz(row);
      b_frag[ni] = B_REGION + row * BN + ((cb ^ swz) << 4) + (lane & 1) * 8;
    }
  }
  // The accumulators, in AGPRs (mfma16_in_place). The MFMAs are asm, whose
  // hazards the compiler does not check, so every write of the accumulators
  // by ordinary code (zeroing) and every read (the epilogue) is separated from
  // the MFMAs by volatile asm in program order: an empty "+a" statement per
  // accumulator pins the value at that point, and s_nop gives the wait states
  // (VALU write -> MFMA srcC read; MFMA write -> VALU / store read).
  v4i acc[MI][NI];
  auto fence_acc = [&]() {
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) asm volatile("" : "+a"(acc[mi][ni]));
  };
  auto zero_acc = [&]() {
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = v4i{0, 0, 0, 0};
    fence_acc();
    asm volatile("s_nop 7\n\ts_nop 7" ::: "memory");
  };
  zero_acc();

  // B reads per slice: lo/hi transposed halves, or whole packed pieces.
  constexpr int BU = PACKED_B ? NI : 2 * NI;
  // One set of A fragments (block mi of the next slice is read right after
  // its last MFMA in this step, 64 slots before it is needed) and two sets of
  // B fragments (every row of MFMAs uses every B block). Row-major B: the two
  // transposed halves land in the low and high pairs of the operand itself.
  v4i fa[MI], fb0[NI], fb1[NI];
  auto read_a = [&](int stage, int mi) {
    fa[mi] = ld_lds_b128(smem + stage * A_BYTES, a_frag[mi]);
  };
  auto read_b = [&](int stage, int u, v4i *fb) {
    const int8_t *Bs = smem + stage * A_BYTES;   // b_frag includes B_REGION
    if constexpr (PACKED_B) {
      fb[u] = ld_lds_b128(Bs, b_frag[u]);
    } else {
      if ((u & 1) == 0) fb[u >> 1].xy = ld_lds_tr8(Bs, b_frag[u >> 1]);
      else fb[u >> 1].zw = ld_lds_tr8(Bs, b_frag[u >> 1] + 8 * BN);
    }
  };
  // The early step's C placement (set per tile) and the wave's strip.
  constexpr int EARLY_STRIPS = (64 - DMAS - 15 + 8) / 8 < 6 ? (64 - DMAS - 15 + 8) / 8 : 6;
  static_assert(8 * EARLY_STRIPS + DMAS <= 63, "vmcnt counts at most 63");
  int32_t *c_tile = nullptr;   // the wave's block of C in the current tile
  LDS_AS int8_t *const lds = (LDS_AS int8_t *)smem;
  constexpr int STRIP0 = NSTAGE * 2 * A_BYTES;
  const StripLanes sl = strip_lanes(lane, STRIP0 + wave * 8192, p.ldc, p.ldd);
  // The 256x128 form's 64-column strip (the first 4 KB of the wave's 8 KB).
  int wb64[4], rb64[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    wb64[k] = STRIP0 + wave * 8192 + strip64_wb(lane, k);
    rb64[k] = STRIP0 + wave * 8192 + strip64_rb(lane, k);
  }
  const uint32_t gofs64 = (uint32_t)(((lane >> 4) * p.ldc + (lane & 15) * 4) * 4);
  const uint32_t gofs64_d = (uint32_t)(((lane >> 4) * p.ldd + (lane & 15) * 4) * 4);
  // One step: MFMAs of slice gs, row by row (odd rows right to left), from fa
  // and fb; slice gs + 1's B blocks go to gb in the first BU slots (block
  // order = first use), its A blocks to fa as each row's last MFMA retires.
  // stg = gs % 4, a compile-time constant at every call.
  // early (compile time; the last step of a tile without D): strips 0 ..
  // EARLY_STRIPS - 1 of the tile's C go out during the step, strip r at slot
  // 8 r + 15, 8 MFMAs after row r's last one, beside the other rows' MFMAs.
  auto step = [&](auto early, int stg, v4i *fb, v4i *gb) {
    constexpr bool EARLY = decltype(early)::value;
    const int s1 = (stg + 1) & 3, s3 = (stg + 3) & 3;
    const int8_t *abase, *bbase;
    next_bases(abase, bbase);   // slice gs + 3
    const uint32_t ma = lds0 + s3 * A_BYTES + wave * DPW * 1024;
    const uint32_t mb = BN == 256 ? ma + B_REGION : lds0 + B_REGION + s3 * A_BYTES + wave * DPW_B * 1024;
    // DMAs every DSTEP slots: 8 of them over 64 slots, or 6 over 32 (every 4)
    constexpr int DSTEP = BN == 256 ? 8 : 4;
#pragma unroll
    for (int slot = 0; slot < MI * NI; ++slot) {
      // Odd rows take their B blocks in reverse ("snake"), so each row's
      // first MFMA reuses the previous one's B operand: 8192^3 1-2 % faster
      // (kernel average, three interleaved rounds on each of two boxes).
      const int mi = slot / NI, pos = slot % NI, ni = (mi & 1) ? NI - 1 - pos : pos;
      mfma16_in_place(acc[mi][ni], fa[mi], fb[ni]);
      if (slot < BU) read_b(s1, slot, gb);
      if (pos == NI - 1) read_a(s1, mi);
      if (slot % DSTEP == 2) {
        const int d = slot / DSTEP;
        if (d < DPW) dma_b128(abase, a_lane[d], ma + d * 1024);
        else if (d < DMAS) dma_b128(bbase, b_lane[d - DPW], mb + (d - DPW) * 1024);
      }
      if constexpr (EARLY) {
        if (slot >= 15 && (slot - 15) % 8 == 0 && (slot - 15) / 8 < EARLY_STRIPS) {
          // The slot barriers keep the strip's AGPR reads here, at least 8
          // MFMAs after row r's last one (tests/test_dma_asm.py checks the
          // distance in the compiled code); a pin (an empty asm redefining
          // the accumulators) made the register allocator spill.
          const int r = (slot - 15) / 8;
          store_strip16_lds<NI, false>(acc[r], c_tile + r * 16 * p.ldc, nullptr, p.ldc, p.ldd, sl, lds);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // Slice gs + 2 has landed (only slice gs + 3's DMAs, and in the early
    // step the strips' 8 stores each, remain in flight; older stores are
    // waited for as well); after the barrier every wave may read it, and
    // stage gs % 4 (read in step gs - 1) may be refilled.
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" :: "n"(DMAS + (EARLY ? 8 * EARLY_STRIPS : 0)) : "memory");
  };
  using Plain = std::integral_constant<bool, false>;
  // EDGE (moved-back tiles, masked stores): no early strips, so no store
  // branch enters the scheduled step; the 256x128 form stores every strip in
  // the epilogue.
  using Early = std::integral_constant<bool, !HAS_D && !EDGE && BN == 256>;

  issue_slice(0);
  issue_slice(1);
  issue_slice(2);
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" :: "n"(DMAS) : "memory");   // slices 0, 1 landed
#pragma unroll
  for (int mi = 0; mi < MI; ++mi) read_a(0, mi);
#pragma unroll
  for (int u = 0; u < BU; ++u) read_b(0, u, fb0);

  int gs = 0;   // global slice index
  for (int it = 0; it < ntiles; ++it) {
    // Kernel-argument scalar loads hoisted by the compiler complete here, not
    // inside the k loop (they retire out of order with LDS reads).
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0); vmcnt, expcnt untouched
    // KT is a multiple of 4 (the host requires K % 256 == 0), so every tile
    // starts at stage 0 with register set 0, and stages and sets rotate
    // statically.
    int bidx, m0, n0, mn, nn;
    tile_coords(it, bidx, m0, n0, mn, nn);
    c_tile = p.C + bidx * p.sc + (int64_t)(m0 + wm * WTM) * p.ldc + n0 + wn * WTN;
    // Without D the tile's last iteration is peeled: its last step stores
    // the first EARLY_STRIPS strips of C (straight-line code: a branch over
    // steps that write the accumulators makes the register allocator
    // shuffle them).
    const int KL = HAS_D || EDGE || BN != 256 ? KT : KT - 4;
    for (int kt = 0; kt < KL; kt += 4, gs += 4) {
      step(Plain(), 0, fb0, fb1);
      step(Plain(), 1, fb1, fb0);
      step(Plain(), 2, fb0, fb1);
      step(Plain(), 3, fb1, fb0);
    }
    if constexpr (!HAS_D && !EDGE && BN == 256) {
      step(Plain(), 0, fb0, fb1);
      step(Plain(), 1, fb1, fb0);
      step(Plain(), 2, fb0, fb1);
      step(Early(), 3, fb1, fb0);
      gs += 4;
    }
    // The last MFMAs' result latency before the epilogue reads any AGPR.
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
    fence_acc();
    // Rows [m0, mn) and columns [n0, nn) of a moved-back tile are its
    // neighbour's to store (0 unless EDGE).
    if constexpr (BN == 256) {
      store_tile16_lds<MI, NI, HAS_D, HAS_D || EDGE ? 0 : EARLY_STRIPS, EDGE>(
          acc, c_tile,
          HAS_D ? p.D + bidx * p.sd + (int64_t)(m0 + wm * WTM) * p.ldd + n0 + wn * WTN : nullptr,
          p.ldc, p.ldd, sl, lds, wm * WTM + (lane >> 5) - (mn - m0),
          wn * WTN + (lane & 31) * 4 >= nn - n0);
    } else {
      const int32_t *d_tile =
          HAS_D ? p.D + bidx * p.sd + (int64_t)(m0 + wm * WTM) * p.ldd + n0 + wn * WTN : nullptr;
      // EDGE: the lane's row in the wave's first strip (4 j + lane / 16 for
      // store j) less the rows the tile leaves to its neighbour, and whether
      // its 4 columns are past the neighbour's.
      const int row_rel0 = wm * WTM + (lane >> 4) - (mn - m0);
      const bool col_ok = wn * WTN + (lane & 15) * 4 >= nn - n0;
#pragma unroll
      for (int mi = 0; mi < MI; ++mi) {
        store_strip64_lds<HAS_D, EDGE>(acc[mi], c_tile + mi * 16 * p.ldc,
                                       HAS_D ? d_tile + mi * 16 * p.ldd : nullptr, p.ldc, p.ldd, wb64,
                                       rb64, gofs64, gofs64_d, lds, row_rel0 + mi * 16, col_ok);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    zero_acc();
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// ---------------------------------------------------------------------------
// Skinny (decode) kernels: M <= 64
// ---------------------------------------------------------------------------

// Row pitch of the LDS-resident A slice in the skinny kernel: a multiple of
// 16 bytes that is 2 (mod 4) chunks, so the 16 rows x 4 chunks read by one
// ds_read_b128 (lane l: row l % 16, chunk l / 16) land on distinct banks in
// every lane group.
__host__ __device__ __forceinline__ int skinny_a_stride(int k_chunk) {
  return k_chunk + 16 * ((2 - (k_chunk >> 4)) & 3);
}

// B stage swizzle of the skinny kernel (rows of 16 chunks): lanes 0-31 of a
// ds_read_b64_tr_b8 read rows r0 + 0..7 and r0 + 16..23 of one chunk, so the
// swizzle gives those 16 rows 16 distinct chunk positions.
__device__ __forceinline__ int skinny_b_swz(int row) {
  return (row & 7) | (((row >> 4) & 1) << 3);
}

struct SkinnyArgs {
  const int8_t *A;
  const int8_t *B;
  const int32_t *D;
  int32_t *C;
  int64_t lda, ldb, ldd, ldc;
  int64_t sa, sb, sd, sc;
  int M, N, K;
  int tiles_n;     // ceil(N / NB)
  int k_split;     // K slices per column slab (workgroups along K)
  int k_chunk;     // rows per slice, a multiple of the stage rows x U
  int32_t *ws;     // [batch][k_split][M][N] partials when k_split > 1
  uint64_t *fin;   // [batch][(M + 1) / 2][N] finishing words (FIN), zero between launches
  int fin_bits;    // FIN: width of each of the word's two sum fields
};

// Finishing word of two K-split output elements (rows 2i and 2i + 1 of one
// column) finished in the kernel. A slice's partial over k_chunk rows of int8
// products lies in [-16256 k_chunk, 16384 k_chunk] (a product lies in
// [-128 * 127, (-128)^2]); biased by 16256 k_chunk it lies in
// [0, 32640 k_chunk]. Each slice adds
//   (1 << 2F) | (biased partial of row 2i + 1) << F | (biased partial of row 2i)
// where F (fin_bits) is the bit length of 32640 k_chunk k_split: both fields
// then stay below 2^F after every add, with no carry between them, and bits
// 2F-63 count the slices that have added; the host needs k_split - 1 < 2^(64-2F).
constexpr int kFinBiasPerRow = 16256;
constexpr int kFinSpanPerRow = 16256 + 16384;

// One workgroup = WAVES waves streams an NB-column slab of B over one K slice.
// Every thread moves one 16-byte chunk per stage, so a stage is R = WAVES*1024/NB
// rows; U stages are in flight in registers. Within a stage, wave w multiplies
// the 64-row k-block w / (NB/16) against n-block w % (NB/16) with one
// v_mfma_i32_16x16x64_i8 (M padded to 16 by zero rows of the LDS-resident A
// slice). At the end the R/64 waves that share an n-block are summed through LDS.
// MB row blocks of 16 (M <= 16 * MB): the A slice holds 16 * MB rows and each
// wave reuses its B fragment for MB MFMAs, one per row block, so B is still
// streamed once for up to 64 rows.
// With a K split the slices' partial sums either go to the workspace for
// skinny_reduce_kernel, or (FIN) are finished here: each slice adds its
// partials of rows 2i and 2i + 1 (biased, in two fields) into their finishing
// word with one agent-scope atomic add, and the slice whose add returns
// k_split - 1 earlier arrivals holds both whole sums (each field of the
// returned word plus its own biased partial, less k_split biases). It writes
// both rows of C (plus D) and stores 0 back into the word. Every step is a
// read-modify-write of that one word, so the word's single modification order
// alone decides which slice is last and what it sees: no fence, no flag in
// other memory, no second kernel.
template <int NB, int WAVES, int U, int MB, bool HAS_D, bool FIN = false>
__global__ __launch_bounds__(64 * WAVES) void skinny_kernel(SkinnyArgs p) {
  constexpr int THREADS = 64 * WAVES;
  constexpr int NBLK = NB / 16;               // 16-column blocks = chunks per row
  constexpr int R = THREADS * 16 / NB;        // rows per stage
  constexpr int KB = R / 64;                  // 64-row k-blocks per stage
  constexpr int STAGE_BYTES = R * NB;
  static_assert(KB * NBLK == WAVES && R % 64 == 0, "one n-block per wave per stage");
  static_assert(NBLK == 16, "skinny_b_swz assumes 256-byte stage rows");
  static_assert(U % 2 == 0, "stages alternate between two LDS buffers by u & 1");
  static_assert(KB == 1 || MB == 1, "the cross-wave sum holds one row block");
  static_assert(!FIN || MB == 1, "finishing in the kernel is instantiated for M <= 16");

  extern __shared__ __attribute__((aligned(16))) int8_t dsmem[];
  const int a_stride = skinny_a_stride(p.k_chunk);
  int8_t *const As = dsmem;
  int8_t *const Bs0 = dsmem + 16 * MB * a_stride;  // stage buffer b at Bs0 + b*STAGE_BYTES

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // XCD-aware order: workgroup w runs on XCD w % 8; give each XCD a contiguous
  // range of (split, slab) indices so slabs that share 128-byte lines of a B
  // row are fetched into the same L2.
  const int total = gridDim.x;
  const int w = blockIdx.x;
  const int q = total >> 3, r = total & 7, x = w & 7;
  const int wl = x * q + (x < r ? x : r) + (w >> 3);
  const int tile = wl % p.tiles_n;
  const int split = wl / p.tiles_n;
  const int bidx = blockIdx.y;
  const int n0 = tile * NB;
  const int M = p.M, N = p.N, K = p.K;
  const int kbeg = split * p.k_chunk;
  // Every slice runs k_chunk/R stages (a multiple of U); rows past K read
  // clamped B rows against zero A columns, so the loop has no data-dependent
  // branches and the compiler keeps U stages of loads in flight.
  const int T = p.k_chunk / R;
  const int8_t *Ab = p.A + bidx * p.sa;
  const int8_t *Bb = p.B + bidx * p.sb;

  const int brow = tid / NBLK, bc = tid % NBLK;
  const int8_t *bsrc = Bb + min(n0 + bc * 16, N - 16);
  const int b_lds = brow * NB + ((bc ^ skinny_b_swz(brow)) << 4);
  // Loads for stages >= T (issued by the last U stages) re-read the slice's
  // last row, which is resident in L2, and are discarded.
  const int krow_last = min(kbeg + p.k_chunk - 1, K - 1);
  // B is streamed exactly once: non-temporal loads keep it from displacing
  // the L2-resident A slice and workspace.
  auto load_stage = [&](int s) -> v4i {
    const int krow = min(kbeg + s * R + brow, krow_last);
    return __builtin_nontemporal_load((const v4i *)(bsrc + (int64_t)krow * p.ldb));
  };
  v4i rb[U];
#pragma unroll
  for (int u = 0; u < U; ++u) rb[u] = load_stage(u);

  // A slice -> LDS, [16 * MB][k_chunk] with zero rows past M and zero k past K.
  {
    const int cpr = p.k_chunk / 16;
    for (int i = tid; i < 16 * MB * cpr; i += THREADS) {
      const int row = i / cpr, c = i - row * cpr;
      const int k = kbeg + c * 16;
      v4i v = v4i{0, 0, 0, 0};
      if (row < M && k < K) v = *(const v4i *)(Ab + (int64_t)row * p.lda + k);
      st_lds_b128(As, row * a_stride + c * 16, v);
    }
  }

  const int g = lane >> 4, j = lane & 15;
  const int nblk = wave % NBLK, kb = wave / NBLK;
  const int r0 = kb * 64 + g * 16 + (j >> 1);
  const int b_frag = r0 * NB + ((nblk ^ skinny_b_swz(r0)) << 4) + (j & 1) * 8;
  const int a_frag = (lane & 15) * a_stride + kb * 64 + g * 16;

  v4i acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = v4i{0, 0, 0, 0};
  for (int t0 = 0; t0 < T; t0 += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = t0 + u;
      int8_t *const Bs = Bs0 + (u & 1) * STAGE_BYTES;
      st_lds_b128(Bs, b_lds, rb[u]);
      rb[u] = load_stage(s + U);
      lds_barrier();
      const v2i lo = ld_lds_tr8(Bs, b_frag);
      const v2i hi = ld_lds_tr8(Bs, b_frag + 8 * NB);
      const v4i b = v4i{lo.x, lo.y, hi.x, hi.y};
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const v4i a = ld_lds_b128(As, a_frag + mb * 16 * a_stride + s * R);
        acc[mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[mb], 0, 0, 0);
      }
    }
  }

  // Sum the KB partials of each n-block through LDS (stage buffers are free
  // after the barrier). 16x16 accumulator layout: element e of lane l is
  // row 4*(l/16) + e, column l%16.
  if constexpr (KB > 1) {
    int32_t *red = (int32_t *)Bs0;
    lds_barrier();
    *(LDS_AS v4i *)((LDS_AS int32_t *)red + (wave * 64 + lane) * 4) = acc[0];
    lds_barrier();
    if (kb != 0) return;
#pragma unroll
    for (int q = 1; q < KB; ++q) {
      const v4i o = *(const LDS_AS v4i *)((const LDS_AS int32_t *)red + ((wave + q * NBLK) * 64 + lane) * 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[0][e] = add_wrap(acc[0][e], o[e]);
    }
  }
  const int col = n0 + nblk * 16 + j;
  if (col >= N) return;
  if (p.k_split == 1) {
    const int32_t *Db = HAS_D ? p.D + bidx * p.sd : nullptr;
    int32_t *Cb = p.C + bidx * p.sc;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = mb * 16 + g * 4 + e;
        if (row < M) {
          int32_t v = acc[mb][e];
          if (HAS_D) v = add_wrap(v, Db[(int64_t)row * p.ldd + col]);
          Cb[(int64_t)row * p.ldc + col] = v;
        }
      }
  } else if constexpr (FIN) {
    // Rows 2i and 2i + 1 share word i of the column: elements e = 0, 1 and
    // e = 2, 3 of the lane.
    const int fw = p.fin_bits;
    const uint64_t field = (1ull << fw) - 1;
    const int64_t bias = (int64_t)kFinBiasPerRow * p.k_chunk;
    uint64_t *fb = p.fin + (int64_t)bidx * ((M + 1) >> 1) * N;
    const int32_t *Db = HAS_D ? p.D + bidx * p.sd : nullptr;
    int32_t *Cb = p.C + bidx * p.sc;
    auto add = [&](int h) {
      const int row = g * 4 + 2 * h;
      // Rows past M hold zero partials (zero A rows), so a lone last row's
      // neighbour field adds the bias alone.
      const uint64_t lo = (uint64_t)((int64_t)acc[0][2 * h] + bias);
      const uint64_t hi = (uint64_t)((int64_t)acc[0][2 * h + 1] + bias);
      return __hip_atomic_fetch_add(fb + (int64_t)(row >> 1) * N + col,
                                    (1ull << (2 * fw)) | (hi << fw) | lo,
                                    __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    auto finish = [&](int h, uint64_t old) {
      const int row = g * 4 + 2 * h;
      if ((old >> (2 * fw)) != (uint64_t)(p.k_split - 1)) return;
      // Each field now holds the sum of k_split biased partials, below 2^fw:
      // the exact sum is that minus k_split biases.
      const int64_t all_bias = bias * p.k_split;
      const int64_t own0 = acc[0][2 * h], own1 = acc[0][2 * h + 1];
      int32_t v0 = (int32_t)((int64_t)(old & field) + own0 + bias - all_bias);
      int32_t v1 = (int32_t)((int64_t)((old >> fw) & field) + own1 + bias - all_bias);
      if (HAS_D) v0 = add_wrap(v0, Db[(int64_t)row * p.ldd + col]);
      Cb[(int64_t)row * p.ldc + col] = v0;
      if (row + 1 < M) {
        if (HAS_D) v1 = add_wrap(v1, Db[(int64_t)(row + 1) * p.ldd + col]);
        Cb[(int64_t)(row + 1) * p.ldc + col] = v1;
      }
      // Every slice has added: the word's last write, which the next launch
      // on the stream sees.
      __hip_atomic_store(fb + (int64_t)(row >> 1) * N + col, 0ull, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    };
    // Up to 8 rows only lanes 0-31 add, and a lane's two adds go out before
    // either result is used, so their round trips overlap (K = 4096,
    // N = 14336, HIP graph, two interleaved rounds on one box: M = 4
    // 12.69-12.70 -> 12.42-12.46 us, M = 8 13.12-13.14 -> 12.80-12.82). With
    // 16 rows every lane adds twice and the adds in flight together queue at
    // the atomic units: one at a time measured 14.06-14.11 against
    // 14.47-14.49 us.
    if (M <= 8) {
      uint64_t old[2] = {0, 0};
#pragma unroll
      for (int h = 0; h < 2; ++h)
        if (g * 4 + 2 * h < M) old[h] = add(h);
#pragma unroll
      for (int h = 0; h < 2; ++h)
        if (g * 4 + 2 * h < M) finish(h, old[h]);
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h)
        if (g * 4 + 2 * h < M) finish(h, add(h));
    }
  } else {
    int32_t *wsb = p.ws + ((int64_t)bidx * p.k_split + split) * M * N;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = mb * 16 + g * 4 + e;
        // Non-temporal: the partials are read once, by the next kernel, and
        // kept out of L2 they need no writeback at the kernel boundary
        // (measured 15.4 -> 15.1 us per decode step at K = 4096, N = 14336).
        if (row < M) __builtin_nontemporal_store(acc[mb][e], wsb + (int64_t)row * N + col);
      }
  }
}

// C = D + sum over the K slices of the skinny partials. Launched on the same
// stream right after skinny_kernel, so stream order makes the partials visible.
struct ReduceArgs {
  const int32_t *ws;   // [batch][k_split][M][N]
  const int32_t *D;
  int32_t *C;
  int64_t ldd, ldc, sd, sc;
  int M, N, k_split;
};

// One wave per workgroup: the sums of a decode step (M = 16: 57344 threads)
// spread over every CU instead of one 256-thread workgroup on each of 224
// (M = 16, K = 4096, N = 14336, 120 graph steps: 14.72 -> 14.65 us; M = 1,
// where 256-thread workgroups covered only 14 CUs: 13.46 -> 13.25 us;
// 128 threads measured between the two, 512 and 1024 slower).
constexpr int kReduceThreads = 64;

template <bool HAS_D>
__global__ __launch_bounds__(kReduceThreads) void skinny_reduce_kernel(ReduceArgs p) {
  const int64_t i = (int64_t)blockIdx.x * kReduceThreads + threadIdx.x;   // over M*N/4 (N % 16 == 0)
  const int64_t per = (int64_t)p.M * p.N / 4;
  if (i >= per) return;
  const int bidx = blockIdx.y;
  const int64_t e = i * 4;
  const int row = (int)(e / p.N), col = (int)(e - (int64_t)row * p.N);
  const int32_t *w = p.ws + (int64_t)bidx * p.k_split * p.M * p.N + e;
  const int64_t slice = (int64_t)p.M * p.N;
  int32_t *c = p.C + bidx * p.sc + (int64_t)row * p.ldc + col;
  v4i s = v4i{0, 0, 0, 0};
  if constexpr (HAS_D) {
    const int32_t *d = p.D + bidx * p.sd + (int64_t)row * p.ldd + col;
#pragma unroll
    for (int t = 0; t < 4; ++t) s[t] = d[t];
  }
  // Up to 8 partials in flight at once: every load of a batch is issued
  // before the first add waits.
  for (int q = 0; q < p.k_split; q += 8) {
    v4i o[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      o[u] = q + u < p.k_split ? __builtin_nontemporal_load((const v4i *)(w + (q + u) * slice))
                               : v4i{0, 0, 0, 0};
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int t = 0; t < 4; ++t) s[t] = add_wrap(s[t], o[u][t]);
  }
#pragma unroll
  for (int t = 0; t < 4; ++t) c[t] = s[t];
}

// ---------------------------------------------------------------------------
// Packed-B decode path
// ---------------------------------------------------------------------------
//
// Packed B: for every 16-column block nb (N/16 of them) and 64-row block kb
// (kbt = ceil(K/64) of them) one 1 KiB tile at byte (nb*kbt + kb)*1024 holds,
// at l*16 + i (lane l = 0..63, i = 0..15), B[kb*64 + 16*(l/16) + i][nb*16 + l%16]
// (zero for rows >= K). That is lane l's operand of v_mfma_i32_16x16x64_i8
// (column l%16, k 16*(l/16)..+15), so a wave feeds the MFMA from one
// coalesced 1 KiB load with no LDS transpose, and each 16-column block is
// contiguous over K.

// Row-major B -> packed B. One workgroup turns a 64-row x 256-column block
// into 16 tiles through LDS: coalesced 16-byte loads in, 16-byte tile chunks out.
struct PackArgs {
  const int8_t *B;
  int8_t *Bp;
  int64_t ldb, sb, sbp;
  int K, N, kbt;
};

__global__ __launch_bounds__(256) void pack_b_kernel(PackArgs p) {
  constexpr int PITCH = 272;   // 256 columns + 16 bytes
  __shared__ __attribute__((aligned(16))) int8_t tile[64 * PITCH];
  const int kb = blockIdx.x, ng = blockIdx.y, bidx = blockIdx.z, tid = threadIdx.x;
  const int8_t *Bb = p.B + bidx * p.sb;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = (tid >> 4) + 16 * i, c = tid & 15;
    const int k = kb * 64 + row, col = ng * 256 + c * 16;
    v4i v = v4i{0, 0, 0, 0};
    if (k < p.K && col < p.N) v = *(const v4i *)(Bb + (int64_t)k * p.ldb + col);
    st_lds_b128(tile, row * PITCH + c * 16, v);
  }
  __syncthreads();
  const int nbt = p.N / 16;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ch = tid + 256 * i, nbl = ch >> 6, l = ch & 63, nb = ng * 16 + nbl;
    if (nb >= nbt) continue;
    v4i v;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t w = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b)
        w |= (uint32_t)(uint8_t)tile[(16 * (l >> 4) + 4 * q + b) * PITCH + nbl * 16 + (l & 15)]
             << (8 * b);
      v[q] = (int)w;
    }
    *(v4i *)(p.Bp + bidx * p.sbp + ((int64_t)nb * p.kbt + kb) * 1024 + l * 16) = v;
  }
}

struct PackedArgs {
  const int8_t *A;
  const int8_t *Bp;
  const int32_t *D;
  int32_t *C;
  int64_t lda, ldd, ldc;
  int64_t sa, sbp, sd, sc;
  int M, N, K;
  int kbt;           // 64-row blocks of the packed layout
  int hpw;           // 8-column half blocks per column group (1 .. 2*NBW)
  int groups;        // column groups: ceil(2 * N/16 / hpw)
  int k_split;       // workgroups along K per column group
  int kb_per_split;  // 64-row blocks per K slice
  int32_t *ws;       // [batch][k_split][M][N] partials when k_split > 1
  uint64_t *fin;     // [batch][(M + 1) / 2][N] finishing words (FIN)
  int fin_bits;      // FIN: width of each of the word's two sum fields
};

// M <= 16 * MB (MB row blocks of 16, up to 64 rows): every B tile a wave loads
// feeds MB MFMAs, so B is streamed once for all of them.
// One workgroup = WAVES waves over one column group and one K slice.
// A column group is hpw consecutive 8-column half blocks, so it touches at
// most NBW 16-column blocks; tiles past its last block are dead and store
// nothing. Whole groups (hpw = 2 * NBW, MASKED false) load every tile, a dead
// tile of the last group re-reading the last block. Smaller groups (MASKED)
// load only live columns: dead tiles load nothing, and with hpw odd the first
// or last block may be live in one half only, whose other half's lanes
// neither load B (a packed tile's half is whole 128-byte lines) nor store C.
// Small groups let a small N spread over every CU without splitting K.
// Wave w takes the 64-row blocks kb_beg + w, kb_beg + w + WAVES, ...;
// per block it loads its MB A fragments (16 bytes per lane, rows past M and k
// past K zero) and the NBW packed B tiles, S blocks ahead of the MFMAs
// (non-temporal loads: B is streamed once). The WAVES partial sums of each
// column block are added through LDS, one row block at a time, and written
// once (plus D), or go to the workspace when K is split across workgroups.
template <int NBW, int WAVES, int S, int MB, bool HAS_D, bool MASKED, bool FIN = false>
__global__ __launch_bounds__(64 * WAVES) void packed_skinny_kernel(PackedArgs p) {
  static_assert(!FIN || MB == 1, "finishing in the kernel is instantiated for M <= 16");
  __shared__ v4i red[WAVES * NBW * 64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // XCD-contiguous logical ids: neighbouring column groups share an L2.
  const int G = gridDim.x, w = blockIdx.x;
  const int q = G >> 3, r = G & 7, x = w & 7;
  const int wl = x * q + (x < r ? x : r) + (w >> 3);
  const int group = wl % p.groups, split = wl / p.groups;
  const int bidx = blockIdx.y;
  const int nbt = p.N / 16;
  const int h0 = group * p.hpw, h1 = min(h0 + p.hpw, 2 * nbt);   // half blocks [h0, h1)
  const int nb0 = h0 >> 1, nb_last = (h1 - 1) >> 1;
  const int kb_beg = split * p.kb_per_split;
  const int kb_end = min(kb_beg + p.kb_per_split, p.kbt);
  const int acol = (lane >> 4) * 16;
  bool arow_ok[MB];
  const int8_t *a_src[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int arow = mb * 16 + (lane & 15);
    arow_ok[mb] = arow < p.M;
    a_src[mb] = p.A + bidx * p.sa + (int64_t)(arow_ok[mb] ? arow : 0) * p.lda + acol;
  }
  const int8_t *Bb = p.Bp + bidx * p.sbp;
  // Tiles 0 .. live-1 are blocks nb0 .. nb_last. Live columns of tile n within
  // its block: [col_lo(n), col_hi(n)); with MASKED a lane loads B only for a
  // live column (l % 16).
  const int live = nb_last - nb0 + 1;
  auto col_lo = [&](int n) { return (MASKED && n == 0 && (h0 & 1)) ? 8 : 0; };
  auto col_hi = [&](int n) { return n >= live ? 0 : (MASKED && n == live - 1 && (h1 & 1)) ? 8 : 16; };
  bool b_live[NBW];
  int64_t b_off[NBW];
#pragma unroll
  for (int n = 0; n < NBW; ++n) {
    b_live[n] = (lane & 15) >= col_lo(n) && (lane & 15) < col_hi(n);
    b_off[n] = (int64_t)min(nb0 + n, nbt - 1) * p.kbt * 1024 + lane * 16;
  }
  v4i acc[MB][NBW];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int n = 0; n < NBW; ++n) acc[mb][n] = v4i{0, 0, 0, 0};

  const int first = kb_beg + wave;
  const int steps = first < kb_end ? (kb_end - first + WAVES - 1) / WAVES : 0;
  v4i a[S][MB], b[S][NBW];
  auto load = [&](int s, v4i (&av)[MB], v4i (&bv)[NBW]) {
    if (s < steps) {
      const int kb = first + s * WAVES;
#pragma unroll
      for (int n = 0; n < NBW; ++n)
        bv[n] = (!MASKED || b_live[n])
                    ? __builtin_nontemporal_load((const v4i *)(Bb + b_off[n] + (int64_t)kb * 1024))
                    : v4i{0, 0, 0, 0};
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        av[mb] = (arow_ok[mb] && kb * 64 + acol < p.K) ? *(const v4i *)(a_src[mb] + kb * 64)
                                                       : v4i{0, 0, 0, 0};
    } else {
#pragma unroll
      for (int n = 0; n < NBW; ++n) bv[n] = v4i{0, 0, 0, 0};
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) av[mb] = v4i{0, 0, 0, 0};
    }
  };
#pragma unroll
  for (int s = 0; s < S; ++s) load(s, a[s], b[s]);
  for (int s0 = 0; s0 < steps; s0 += S) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int n = 0; n < NBW; ++n)
          acc[mb][n] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[s][mb], b[s][n], acc[mb][n], 0, 0, 0);
      load(s0 + s + S, a[s], b[s]);
    }
  }

  // 16x16 accumulator layout: element e of lane l is row 4*(l/16) + e,
  // column l%16. Thread t sums output (block t/256, row (t/16)%16, column t%16)
  // over the waves, so 16 consecutive threads write 64 contiguous bytes.
  // One row block at a time through the same LDS buffer.
  const int32_t *Db = HAS_D ? p.D + bidx * p.sd : nullptr;
  int32_t *Cb = p.C + bidx * p.sc;
  if constexpr (FIN) {
    // K slices finished here through the skinny kernel's finishing words
    // (rows 2i and 2i + 1 of a column share one; see kFinBiasPerRow): thread
    // t sums rows 2 pr and 2 pr + 1 of column c of block n over the waves,
    // so 16 consecutive threads add into one 128-byte line of words.
#pragma unroll
    for (int n = 0; n < NBW; ++n) red[(wave * NBW + n) * 64 + lane] = acc[0][n];
    __syncthreads();
    const int fw = p.fin_bits;
    const uint64_t field = (1ull << fw) - 1;
    const int64_t bias = (int64_t)kFinBiasPerRow * p.kb_per_split * 64;
    uint64_t *fb = p.fin + (int64_t)bidx * ((p.M + 1) >> 1) * p.N;
    for (int t = tid; t < NBW * 128; t += 64 * WAVES) {
      const int n = t >> 7, pr = (t >> 4) & 7, c = t & 15;
      const int row = 2 * pr, src = (row >> 2) * 16 + c, e = row & 3;
      int32_t s0 = 0, s1 = 0;
#pragma unroll
      for (int wv = 0; wv < WAVES; ++wv) {
        const int32_t *v = (const int32_t *)&red[(wv * NBW + n) * 64 + src];
        s0 = add_wrap(s0, v[e]);
        s1 = add_wrap(s1, v[e + 1]);
      }
      if (MASKED ? (c < col_lo(n) || c >= col_hi(n)) : n >= live) continue;
      if (row >= p.M) continue;
      const int col = (nb0 + n) * 16 + c;
      // Rows past M hold zero sums (zero A rows): a lone last row's
      // neighbour field adds the bias alone.
      const uint64_t lo = (uint64_t)((int64_t)s0 + bias), hi = (uint64_t)((int64_t)s1 + bias);
      uint64_t *word = fb + (int64_t)pr * p.N + col;
      const uint64_t old = __hip_atomic_fetch_add(word, (1ull << (2 * fw)) | (hi << fw) | lo,
                                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if ((old >> (2 * fw)) != (uint64_t)(p.k_split - 1)) continue;
      const int64_t all_bias = bias * p.k_split;
      int32_t v0 = (int32_t)((int64_t)((old & field) + lo) - all_bias);
      int32_t v1 = (int32_t)((int64_t)(((old >> fw) & field) + hi) - all_bias);
      if (HAS_D) v0 = add_wrap(v0, Db[(int64_t)row * p.ldd + col]);
      Cb[(int64_t)row * p.ldc + col] = v0;
      if (row + 1 < p.M) {
        if (HAS_D) v1 = add_wrap(v1, Db[(int64_t)(row + 1) * p.ldd + col]);
        Cb[(int64_t)(row + 1) * p.ldc + col] = v1;
      }
      __hip_atomic_store(word, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return;
  }
  int32_t *wsb = p.ws ? p.ws + ((int64_t)bidx * p.k_split + split) * p.M * p.N : nullptr;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    if (mb > 0) __syncthreads();   // the previous row block's sums are read
#pragma unroll
    for (int n = 0; n < NBW; ++n) red[(wave * NBW + n) * 64 + lane] = acc[mb][n];
    __syncthreads();
    for (int t = tid; t < NBW * 256; t += 64 * WAVES) {
      const int n = t >> 8, r16 = (t >> 4) & 15, c = t & 15;
      const int src = (r16 >> 2) * 16 + c, e = r16 & 3;
      int32_t s = 0;
#pragma unroll
      for (int wv = 0; wv < WAVES; ++wv)
        s = add_wrap(s, ((const int32_t *)&red[(wv * NBW + n) * 64 + src])[e]);
      const int row = mb * 16 + r16;
      if (MASKED ? (c < col_lo(n) || c >= col_hi(n)) : n >= live) continue;
      if (row >= p.M) continue;
      const int col = (nb0 + n) * 16 + c;
      if (p.k_split == 1) {
        if (HAS_D) s = add_wrap(s, Db[(int64_t)row * p.ldd + col]);
        Cb[(int64_t)row * p.ldc + col] = s;
      } else {
        __builtin_nontemporal_store(s, wsb + (int64_t)row * p.N + col);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Generic kernel: any shape, stride and alignment
// ---------------------------------------------------------------------------

struct GenericArgs {
  const int8_t *A;
  const int8_t *B;
  const int32_t *D;
  int32_t *C;
  int64_t lda, ldb, ldd, ldc;
  int64_t sa, sb, sd, sc;
  int64_t M, N, K, batch;
};

__global__ __launch_bounds__(256) void generic_kernel(GenericArgs p) {
  const int64_t j = (int64_t)blockIdx.x * 64 + (threadIdx.x & 63);
  if (j >= p.N) return;
  for (int64_t b = blockIdx.z; b < p.batch; b += gridDim.z) {
    const int8_t *Ab = p.A + b * p.sa;
    const int8_t *Bb = p.B + b * p.sb;
    for (int64_t i = (int64_t)blockIdx.y * 4 + (threadIdx.x >> 6); i < p.M;
         i += (int64_t)gridDim.y * 4) {
      uint32_t s = p.D ? (uint32_t)p.D[b * p.sd + i * p.ldd + j] : 0u;
      const int8_t *arow = Ab + i * p.lda;
      const int8_t *bcol = Bb + j;
      int64_t t = 0;
      // 32 independent loads of A and B per step, so their latencies overlap
      for (; t + 32 <= p.K; t += 32) {
        int32_t av[32], bv[32];
#pragma unroll
        for (int u = 0; u < 32; ++u) {
          av[u] = arow[t + u];
          bv[u] = bcol[(t + u) * p.ldb];
        }
#pragma unroll
        for (int u = 0; u < 32; ++u) s += (uint32_t)(av[u] * bv[u]);
      }
      if (t + 16 <= p.K) {
        int32_t av[16], bv[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          av[u] = arow[t + u];
          bv[u] = bcol[(t + u) * p.ldb];
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) s += (uint32_t)(av[u] * bv[u]);
        t += 16;
      }
      for (; t < p.K; ++t) s += (uint32_t)((int32_t)arow[t] * (int32_t)bcol[t * p.ldb]);
      p.C[b * p.sc + i * p.ldc + j] = (int32_t)s;
    }
  }
}

// ---------------------------------------------------------------------------
// Gemmini command-stream replay
// ---------------------------------------------------------------------------

// One workgroup of 256 threads executes the lowered stream in order, one
// 16 x 16 tile operation at a time (thread t owns element (t / 16, t % 16)),
// with the scratchpad, the accumulator and the latched B tile in LDS and a
// barrier between operations. Every address is checked against the declared
// sizes before use; the first failure is recorded and ends the replay.
struct ReplayArgs {
  const int32_t *prog;
  int n_ops;
  const int8_t *A;
  const int8_t *B;
  int32_t *C;
  int64_t size_a, size_b, size_c;
  int spad_rows, acc_rows;
  int32_t *status;
};

__global__ __launch_bounds__(256) void replay_kernel(ReplayArgs p) {
  extern __shared__ __attribute__((aligned(16))) int8_t lds[];
  int8_t *const spad = lds;                                            // [spad_rows][16]
  int32_t *const acc = (int32_t *)(lds + (int64_t)p.spad_rows * 16);   // [acc_rows][16]
  int8_t *const latch = (int8_t *)(acc + (int64_t)p.acc_rows * 16);   // [16][16]
  __shared__ int err[4];
  const int t = threadIdx.x, r = t >> 4, c = t & 15;
  if (t == 0) err[0] = err[1] = err[2] = err[3] = 0;
  __syncthreads();
  auto fail_at = [&](int code, int index) {
    if (atomicCAS(&err[0], 0, code) == 0) {
      err[1] = index;
      err[2] = r;
      err[3] = c;
    }
  };
  for (int i = 0; i < p.n_ops; ++i) {
    const int32_t *w = p.prog + 8 * (int64_t)i;
    const int op = w[0], index = w[7];
    if (op == VT_REPLAY_MVIN) {
      const int64_t off = w[2], stride = w[3];
      const int row = w[4];
      const int64_t size = w[1] ? p.size_b : p.size_a;
      if (row < 0 || row > p.spad_rows - 16 || off < 0 || stride < 0 || off + 15 * stride + 16 > size)
        fail_at(VT_REPLAY_STATUS_RANGE, index);
      else
        spad[(row + r) * 16 + c] = (w[1] ? p.B : p.A)[off + r * stride + c];
    } else if (op == VT_REPLAY_LATCH_B) {
      const int row = w[1];
      if (row < 0 || row > p.spad_rows - 16) fail_at(VT_REPLAY_STATUS_RANGE, index);
      else latch[t] = spad[row * 16 + t];
    } else if (op == VT_REPLAY_COMPUTE) {
      const int arow = w[1], orow = w[2];
      if (arow < 0 || arow > p.spad_rows - 16 || orow < 0 || orow > p.acc_rows - 16) {
        fail_at(VT_REPLAY_STATUS_RANGE, index);
      } else {
        int32_t s = 0;
#pragma unroll
        for (int q = 0; q < 16; ++q) s += (int32_t)spad[(arow + r) * 16 + q] * (int32_t)latch[q * 16 + c];
        const int64_t v = (int64_t)s + (w[3] ? acc[(orow + r) * 16 + c] : 0);
        if (v < INT32_MIN || v > INT32_MAX) fail_at(VT_REPLAY_STATUS_OVERFLOW, index);
        else acc[(orow + r) * 16 + c] = (int32_t)v;
      }
    } else if (op == VT_REPLAY_MVOUT) {
      const int orow = w[1];
      const int64_t off = w[2], ldc = w[3];
      if (orow < 0 || orow > p.acc_rows - 16 || off < 0 || ldc < 16 || off + 15 * ldc + 16 > p.size_c)
        fail_at(VT_REPLAY_STATUS_RANGE, index);
      else
        p.C[off + r * ldc + c] = acc[(orow + r) * 16 + c];
    } else {
      fail_at(VT_REPLAY_STATUS_OPCODE, index);
    }
    __syncthreads();
    if (err[0]) break;
  }
  if (t < 4) p.status[t] = err[t];
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

thread_local std::string g_err;

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

#define VT_HIP_CHECK(expr)                                                     \
  do {                                                                         \
    hipError_t e_ = (expr);                                                    \
    if (e_ != hipSuccess)                                                      \
      return fail(VT_EHIP, "%s failed: %s", #expr, hipGetErrorString(e_));    \
  } while (0)

struct VariantInfo {
  const char *name;
  int tile_m, tile_n, tile_k, threads, lds_bytes;
};

// lds_bytes of the MFMA variants is that of their tile kernel
// (gemm_mfma_kernel, 3 slice buffers); the persistent 256x256 kernels take
// kDma16Lds or kDmaLds per workgroup, one workgroup per CU. lds_bytes of the
// skinny variants excludes the A slice (16 x (k_chunk+16)), which depends on
// K and the split.
const VariantInfo kVariants[VT_VARIANT_COUNT] = {
    {"auto", 0, 0, 0, 0, 0},
    {"mfma_256x256", 256, 256, 64, 256, 3 * (256 * 64 + 64 * 256)},
    {"mfma_128x128", 128, 128, 64, 256, 3 * (128 * 64 + 64 * 128)},
    {"skinny", 16, 256, 64, 1024, 2 * 16 * 1024},
    {"generic", 4, 64, 1, 256, 0},
    {"mfma_256x128", 256, 128, 64, 256, 3 * (256 * 64 + 64 * 128)},
    {"padded", 16, 16, 16, 256, 0},   // padding granularity; the inner kernel decides the rest
};

// Default skinny configuration: 256-column slabs (full 128-byte lines of B
// per row), 16 waves, 2 stages in flight per thread.
constexpr int kSkinnyNB = 256, kSkinnyWaves = 16, kSkinnyU = 2;
// Rows the skinny kernel takes: up to 4 row blocks of 16.
constexpr int kSkinnyMaxM = 64;
// Up to this many rows (one row block) a K-split skinny launch finishes its
// sums in the kernel (skinny_kernel FIN) instead of a second launch. K = 4096,
// N = 14336, four slices, HIP graph of 120 steps over 10 input sets, three
// interleaved rounds on one box, finishing against the second launch: M = 2
// 11.93 against 12.39-12.46 us, M = 4 12.66-12.73 against 13.59-13.63, M = 8
// 13.08-13.10 against 14.09-14.13, M = 12 13.43-13.49 against 14.40-14.46,
// M = 16 14.10-14.12 against 14.70-14.78. With one word per element (one
// atomic per element and slice) finishing had lost from 8 rows (M = 8 14.6,
// M = 16 16.7 us); a word per two rows halves the atomics.
constexpr int kSkinnyFinMaxM = 16;
// Row blocks of 16 the skinny kernel is instantiated with for M rows.
int skinny_row_blocks(int64_t M) { return M <= 16 ? 1 : M <= 32 ? 2 : 4; }
// LDS for the replay's scratchpad and accumulator (plus the latched B tile).
constexpr int kMaxReplayLds = 152 * 1024;
constexpr int kMaxSkinnyLds = 160 * 1024;

// Scratch memory of one call: the K-split partial sums of the decode
// kernels and the padded variant's operand copies.
enum ScratchKind { kPartials = 0, kPadded = 1, kFinWords = 2, kScratchKinds = 3 };

struct Workspace {
  void *ptr = nullptr;
  size_t bytes = 0;
};

struct DeviceState {
  bool probed = false;
  bool ok = false;
  int num_cus = 256;
  std::string arch;
  hipError_t attr_err = hipSuccess;   // dynamic-LDS limits, set once on this device
  std::map<void *, Workspace> ws[kScratchKinds];   // per stream, per kind
  // Workspaces superseded by larger ones. They are never freed: a HIP graph
  // captured earlier may still hold their addresses, and a host thread may
  // still be launching with one.
  std::vector<void *> retired;
  int8_t *scratch = nullptr;   // this device's address of the static scratch array
  hipError_t scratch_err = hipSuccess;
};

std::mutex g_mu;
std::map<int, DeviceState> g_dev;

void set_kernel_attributes(DeviceState &st);

int current_device(int *dev_out, DeviceState **st_out) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0)
    return fail(VT_ENODEV, "no HIP device available");
  int dev = 0;
  VT_HIP_CHECK(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lk(g_mu);
  DeviceState &st = g_dev[dev];
  if (!st.probed) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess)
      return fail(VT_ENODEV, "hipGetDeviceProperties(%d) failed", dev);
    st.arch = prop.gcnArchName;
    st.num_cus = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
    st.ok = strncmp(prop.gcnArchName, "gfx950", 6) == 0;
    // Kernel attributes and the address of the static scratch array belong
    // to a device: set up here, once per device, with that device current.
    if (st.ok) {
      set_kernel_attributes(st);
      void *ptr = nullptr;
      st.scratch_err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
      st.scratch = st.scratch_err == hipSuccess ? (int8_t *)ptr : nullptr;
    }
    st.probed = true;
  }
  if (!st.ok)
    return fail(VT_ENODEV, "device %d is %s; this library is built for gfx950", dev,
                st.arch.c_str());
  if (st.attr_err != hipSuccess)
    return fail(VT_EHIP, "hipFuncSetAttribute (dynamic LDS) failed on device %d: %s", dev,
                hipGetErrorString(st.attr_err));
  *dev_out = dev;
  *st_out = &st;
  return VT_OK;
}

// The library's workspace of one kind on (device, stream). Calls on one
// stream are ordered, so a stream's workspace is never used by two launches
// in flight. It only grows, at least doubling, and is allocated outside
// stream capture only: a call that needs more than the stream has while the
// stream is being captured is refused (run it once before capturing).
int get_workspace(DeviceState *st, void *stream, ScratchKind kind, size_t bytes, void **out) {
  std::lock_guard<std::mutex> lk(g_mu);
  Workspace &w = st->ws[kind][stream];
  if (w.bytes < bytes) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    VT_HIP_CHECK(hipStreamIsCapturing((hipStream_t)stream, &cs));
    if (cs != hipStreamCaptureStatusNone)
      return fail(VT_EUNSUPPORTED,
                  "this call needs %zu bytes of workspace and the stream, which is being "
                  "captured, has %zu: make the same call once on this stream before capture",
                  bytes, w.bytes);
    size_t nb = bytes > 2 * w.bytes ? bytes : 2 * w.bytes;
    if (nb < (1u << 20)) nb = 1u << 20;
    void *p = nullptr;
    VT_HIP_CHECK(hipMalloc(&p, nb));
    // Finishing words read zero before their first launch, and every launch
    // leaves them zero. The clear is ordered before that launch on the same
    // stream; it is never captured, since growth under capture is refused above.
    if (kind == kFinWords) VT_HIP_CHECK(hipMemsetAsync(p, 0, nb, (hipStream_t)stream));
    if (w.ptr) st->retired.push_back(w.ptr);
    w.ptr = p;
    w.bytes = nb;
  }
  *out = w.ptr;
  return VT_OK;
}

// Where a call's scratch memory comes from: the per-stream workspaces above,
// or consecutive 256-byte aligned pieces of a fixed device buffer of
// kScratchBytes.
constexpr size_t kScratchBytes = (size_t)32 << 20;
static_assert(sizeof(scratch) == kScratchBytes, "the fixed scratch buffer is the static array");

struct Scratch {
  DeviceState *st = nullptr;
  void *stream = nullptr;
  int8_t *fixed = nullptr;   // device address of `scratch`, or null
  size_t used = 0;

  int take(ScratchKind kind, size_t bytes, void **out) {
    if (!fixed) return get_workspace(st, stream, kind, bytes, out);
    const size_t need = (bytes + 255) / 256 * 256;
    if (need > kScratchBytes - used)
      return fail(VT_EUNSUPPORTED,
                  "this call needs %zu bytes of scratch and the fixed scratch buffer holds %zu",
                  used + need, kScratchBytes);
    *out = fixed + used;
    used += need;
    return VT_OK;
  }
};

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// Byte range [lo, hi) a [batch][rows][ld] operand of `elem`-byte elements
// touches when `cols` columns of each row are used (batch stride `stride`,
// 0 = one matrix shared by every batch). Sizes are bounded by the caller;
// the products are formed in 128 bits and must stay below 2^56 bytes.
struct Extent {
  uintptr_t lo = 0, hi = 0;
};
bool operand_extent(const void *p, int64_t batch, int64_t stride, int64_t rows, int64_t ld,
                    int64_t cols, int64_t elem, Extent *out) {
  const __int128 last = (__int128)(batch - 1) * stride + (__int128)(rows - 1) * ld + cols;
  const __int128 bytes = last * elem;
  if (bytes < 0 || bytes >= ((__int128)1 << 56)) return false;
  out->lo = (uintptr_t)p;
  out->hi = (uintptr_t)p + (uintptr_t)bytes;
  return out->hi >= out->lo;
}

bool overlaps(const Extent &a, const Extent &b) { return a.lo < b.hi && b.lo < a.hi; }

// The output may not share memory with an input, except that D may be C
// itself (same base, leading dimension and batch stride: in-place C = C + A.B).
// Every lane reads its inputs and writes its own outputs with no ordering
// against other lanes, so any other overlap would race.
int check_operand_overlap(const void *A, const void *B, const int32_t *D, const int32_t *C,
                          int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb_rows,
                          int64_t ldb, int64_t b_cols, int64_t ldd, int64_t ldc, int64_t batch,
                          int64_t sa, int64_t sb, int64_t sd, int64_t sc, const char *who) {
  Extent ec, ea, eb, ed;
  if (!operand_extent(C, batch, sc, M, ldc, N, 4, &ec))
    return fail(VT_EINVAL, "%s: C extent beyond 2^56 bytes", who);
  if (K > 0) {
    if (!operand_extent(A, batch, sa, M, lda, K, 1, &ea) ||
        !operand_extent(B, batch, sb, ldb_rows, ldb, b_cols, 1, &eb))
      return fail(VT_EINVAL, "%s: A or B extent beyond 2^56 bytes", who);
    if (overlaps(ec, ea) || overlaps(ec, eb))
      return fail(VT_EINVAL, "%s: C overlaps A or B in memory", who);
  }
  if (D) {
    if (!operand_extent(D, batch, sd, M, ldd, N, 4, &ed))
      return fail(VT_EINVAL, "%s: D extent beyond 2^56 bytes", who);
    const bool in_place = (const void *)D == (const void *)C && ldd == ldc && (batch == 1 || sd == sc);
    if (!in_place && overlaps(ec, ed))
      return fail(VT_EINVAL, "%s: D overlaps C without being C itself (same ld and stride)", who);
  }
  return VT_OK;
}

struct Problem {
  const int8_t *A;
  const int8_t *B;
  const int32_t *D;
  int32_t *C;
  int64_t M, N, K, lda, ldb, ldd, ldc, batch, sa, sb, sd, sc;
};

bool vector_ok(const Problem &q) {
  return q.N % 16 == 0 && q.K % 16 == 0 && q.K > 0 && q.lda % 16 == 0 &&
         q.ldb % 16 == 0 && q.sa % 16 == 0 && q.sb % 16 == 0 && aligned16(q.A) &&
         aligned16(q.B) && q.M < (1ll << 30) && q.N < (1ll << 30) && q.K < (1ll << 30);
}

// Workgroups along K for the skinny kernel: 1 when the column slabs alone
// give most CUs a workgroup, else enough slices for ~224 workgroups, each at
// least one unrolled pipeline (stage rows x U) long.
int choose_k_split(int64_t N, int64_t K, int64_t batch) {
  const int64_t tiles = (N + kSkinnyNB - 1) / kSkinnyNB * batch;
  if (tiles >= 192) return 1;
  const int64_t pipe = (int64_t)kSkinnyWaves * 1024 / kSkinnyNB * kSkinnyU;
  int64_t ks = (224 + tiles - 1) / tiles;
  const int64_t max_by_k = (K + pipe - 1) / pipe;
  if (ks > max_by_k) ks = max_by_k;
  if (ks < 1) ks = 1;
  if (ks > 64) ks = 64;
  return (int)ks;
}

// Shapes the padded path takes: padded sizes the vector kernels accept. Auto
// selection takes it from 3 * 2^24 multiply-adds: below that the VALU
// kernel is faster than one copy launch, the product and the copy-out.
bool padded_fits(const Problem &q) {
  return q.K > 0 && q.M < (1ll << 30) && q.N + 15 < (1ll << 30) && q.K + 15 < (1ll << 30) &&
         q.batch <= 65535;
}

// The MFMA kernels address A and B from 64-bit bases at each tile's origin
// plus 32-bit lane offsets within one tile (256 rows of A, 64 rows of B).
bool mfma_addressable(const Problem &q) {
  return (__int128)256 * q.lda < (1ll << 32) - 4096 && (__int128)64 * q.ldb < (1ll << 32) - 4096;
}

int launch_generic(const Problem &q, hipStream_t stream);

int select_variant(const Problem &q, bool vec, int32_t *variant, int32_t *k_split) {
  *k_split = 0;
  if (!vec || q.K == 0) {
    const double macs = (double)q.M * (double)q.N * (double)q.K * (double)q.batch;
    *variant = (padded_fits(q) && macs >= 50331648.0) ? VT_VARIANT_PADDED : VT_VARIANT_GENERIC;
    return VT_OK;
  }
  // Tiny problems past the skinny kernel's rows: with K <= 64 the VALU
  // kernel's K loop is at most two batches of loads, under the MFMA kernels'
  // fixed cost (64^3: 2.4 us against 4.3 us per launch in a HIP graph; from
  // 128^3 on the MFMA kernel is faster).
  if (q.M > 16 && q.K <= 64 &&
      (double)q.M * (double)q.N * (double)q.K * (double)q.batch <= 1048576.0) {
    *variant = VT_VARIANT_GENERIC;
    return VT_OK;
  }
  if (q.M <= 16) {
    *variant = VT_VARIANT_SKINNY;
    *k_split = choose_k_split(q.N, q.K, q.batch);
    return VT_OK;
  }
  // 17..64 rows: streaming B once on the skinny kernel (2 or 4 row blocks)
  // beats the MFMA tiles' long K loop unless 128-column tiles alone fill the
  // chip (measured at K = 4096: 1.5-3x faster for N = 4096 .. 28672, even at
  // N = 57344 and 65536; 7x at N = 1024, K = 16384). Short K stays on the
  // MFMA kernels, whose K loop is then a round trip or two.
  if (q.M <= kSkinnyMaxM && q.K >= 512 && (q.N + 127) / 128 * q.batch < 256) {
    *variant = VT_VARIANT_SKINNY;
    *k_split = choose_k_split(q.N, q.K, q.batch);
    return VT_OK;
  }
  // Rows too long for the MFMA kernels' tile-relative 32-bit offsets
  // (lda >= 2^24 bytes) go to the VALU kernel.
  if (!mfma_addressable(q)) {
    *variant = VT_VARIANT_GENERIC;
    return VT_OK;
  }
  // Batched B-reuse with contiguous batches is one GEMM with stacked M.
  const bool fold = q.batch > 1 && q.sb == 0 && q.sa == q.M * q.lda && q.sc == q.M * q.ldc &&
                    (!q.D || q.sd == q.M * q.ldd);
  const int64_t m_eff = fold ? q.M * q.batch : q.M;
  const int64_t b_eff = fold ? 1 : q.batch;
  const int64_t t256 = (m_eff + 255) / 256 * ((q.N + 255) / 256) * b_eff;
  // Below a full round of 256x256 tiles, the persistent kernel (K whole
  // 64-deep slices, M, N >= 256) wins from more than half a round when K is
  // long: N = 4096, K = 4096, 160 tiles 49.2 us against 59.3 (128x128) and
  // 61.9 (256x128), 224 tiles 56.3 against 70.7; at 128 tiles 256x128 is
  // ahead (43.0 against 46.8 us). With K = 1024 it wins only near a full
  // round (224 tiles 24.7-25.9 us against 26.2-27.6; 192 tiles 23.1-25.3
  // against 23.1-23.2 on 128x128), and at K <= 1024 128x128 beats 256x128
  // (K = 512, 144-168 tiles: 14.8-15.0 us against 16.9-17.4). With K >= 4096
  // 256x128 also wins at 192 of its tiles (96 of 256x256; M = 1536, N = 4096:
  // 36.1 against 38.7 us, K = 8192 64.8 against 71.7).
  // From K = 12288 the persistent kernel, K split in four, also wins at 40-96
  // tiles (M x N x K: 1280 x 2048 x 16384 54.2 us against 73.9 on 128x128;
  // 768 x 4096 x 12288 51.9 against 57.9; 512 x 8192 x 16384 79.5 against
  // 112.5), and from K = 32768 at 97-128 tiles as well (2048 x 4096 x 32768
  // 221.8 against 294.5 on 256x128).
  const bool persistent = q.K % 64 == 0 && m_eff >= 256 && q.N >= 256;
  const int64_t t128 = (m_eff + 255) / 256 * ((q.N + 127) / 128) * b_eff;
  if ((t256 >= 256 && q.N >= 256) ||
      (persistent && ((q.K >= 2048 && t256 > 128) || (q.K >= 1024 && t256 > 192) ||
                      (q.K >= 12288 && t256 >= 40 && (t256 <= 96 || q.K >= 32768))))) {
    *variant = VT_VARIANT_MFMA_256x256;
  } else {
    // M >= 256, N >= 128 and K % 256 == 0 run on the persistent kernel's
    // 256x128 form, which wins over 128x128 tiles from more than half a round
    // of its tiles at K >= 1024 (M x N: 1280 x 4096, K = 1024 12.8 us against
    // 14.0, K = 4096 29.8 against 37.3; 2560 x 2048, K = 2048 18.5 against
    // 22.0; 768 x 8192, K = 2048 19.5 against 23.3; 512 x 14336, K = 2048 20.8
    // against 24.6; ragged: 1200 x 4096 x 1024 12.6 against 14.2, 500 x 14336
    // x 2048 21.4 against 24.2), but not at half a round or less (1024 x 4096
    // x 4096: 28.8 against 25.2), except at 48-64 tiles from K = 12288, K
    // split in four (768 x 2048 x 16384 37.2 against 45.6; 1024 x 2048 x
    // 32768 71.6 against 88.1).
    const bool form128 = m_eff >= 256 && q.N >= 128 && q.K % 256 == 0;
    const bool wide = (q.K >= 2048 && (t128 >= 256 || (q.K >= 4096 && t128 >= 192))) ||
                      (form128 && q.K >= 1024 && t128 > 128 && t128 <= 256) ||
                      (form128 && q.K >= 12288 && t128 >= 48 && t128 <= 64);
    *variant = (wide && m_eff >= 256) ? VT_VARIANT_MFMA_256x128 : VT_VARIANT_MFMA_128x128;
  }
  return VT_OK;
}


// Waves per workgroup of the persistent 256x256 kernel.
constexpr int kDmaWaves = 4;

// Persistent 256x256 problems run on gemm_dma16_kernel (16x16x64) when K is a whole
// number of 256-deep groups of four slices and its epilogue's 16-byte C and D
// accesses are aligned (C, D 16-byte aligned; ldc, ldd and the batch strides
// multiples of 4 elements, ldc and ldd below 2^29); otherwise on
// gemm_dma_kernel (32x32x32, 4-byte stores, 64-bit row addresses). Measured per launch (HIP graphs, two passes), 16x16x64 against
// 32x32x32 at 8192 x 8192 x K: K = 256 58-61 against 62-63 us, 1024 91-99
// against 99, 2048 139-145 against 149-150, 4096 226-229 against 245-249,
// 8192 400 against 447, 8192 with D 459 against 518; config 3 (K = 1024) 46-49
// against 49; 4096^3 60-69 against 66-67.
bool use_dma16(const Problem &r) {
  // The epilogue also addresses a lane's 16 bytes as a 32-bit byte offset
  // from its row pair's base (one row of ldc or ldd plus 512 bytes).
  const bool c_ok = aligned16(r.C) && r.ldc % 4 == 0 && (r.batch == 1 || r.sc % 4 == 0) &&
                    r.ldc < (1ll << 29);
  const bool d_ok = !r.D || (aligned16(r.D) && r.ldd % 4 == 0 && (r.batch == 1 || r.sd % 4 == 0) &&
                             r.ldd < (1ll << 29));
  return r.K % 256 == 0 && c_ok && d_ok;
}

// Row-major problems of M >= 256 and N >= 128 run on the 256x128 form of
// gemm_dma16_kernel (persistent, one workgroup per CU; a last tile row or
// column past M or N moved back to end there, its EDGE instantiation storing
// only what its neighbour does not) when its 16-byte C and D accesses are
// aligned; it addresses a lane's 16 bytes from its 4-row group's base (three
// rows of ldc or ldd plus 256 bytes) as a 32-bit byte offset. Otherwise
// gemm_mfma_kernel<256, 128> takes them.
bool dma16_128_fits(const Problem &r) {
  return r.K > 0 && r.M >= 256 && r.N >= 128 && r.ldc < (1ll << 28) &&
         (!r.D || r.ldd < (1ll << 28)) && use_dma16(r);
}

template <int BM, int BN, int EDGE, bool HAS_D, bool PACKED>
void launch_mfma_kernel(bool short_k, bool early_d, dim3 grid, dim3 block, hipStream_t stream,
                        const GemmArgs &a) {
  if constexpr (HAS_D) {
    if (early_d) {
      if (short_k) hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, EDGE, true, true, true, PACKED>), grid, block, 0, stream, a);
      else hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, EDGE, true, false, true, PACKED>), grid, block, 0, stream, a);
      return;
    }
  }
  if (short_k) hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, EDGE, HAS_D, true, false, PACKED>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, EDGE, HAS_D, false, false, PACKED>), grid, block, 0, stream, a);
}

// Contiguous shared-B batches as one GEMM with stacked M.
Problem mfma_fold(const Problem &q) {
  Problem r = q;
  if (r.batch > 1 && r.sb == 0 && r.sa == r.M * r.lda && r.sc == r.M * r.ldc &&
      (!r.D || r.sd == r.M * r.ldd) && r.M * r.batch < (1ll << 30)) {
    r.M *= r.batch;
    r.batch = 1;
  }
  return r;
}

// C = D + the k_split partial sums in ws, on `stream` after the kernel that
// wrote them (stream order publishes the partials).
int launch_reduce(const ReduceArgs &r, int64_t batch, hipStream_t stream) {
  const int64_t per = (int64_t)r.M * r.N / 4;
  if (per > 0x7fffffff || batch > 65535) return fail(VT_EUNSUPPORTED, "reduction grid too large");
  dim3 grid((unsigned)((per + kReduceThreads - 1) / kReduceThreads), (unsigned)batch);
  if (r.D) hipLaunchKernelGGL(skinny_reduce_kernel<true>, grid, dim3(kReduceThreads), 0, stream, r);
  else hipLaunchKernelGGL(skinny_reduce_kernel<false>, grid, dim3(kReduceThreads), 0, stream, r);
  VT_HIP_CHECK(hipGetLastError());
  return VT_OK;
}

// K slices for an MFMA launch whose tiles alone would leave most of the chip
// idle: a K of at least 1024 over at most 64 tiles is cut into ks slices of
// whole 128-deep steps, each at least 512 deep, for up to 256 workgroups. The
// slices run as ks batches of the same kernel into a partial-sum workspace
// and skinny_reduce_kernel adds them (and D). The partial sums cost
// 8 * ks * M * N bytes of traffic, which a split of two over 65..128 tiles
// does not earn back (M = 128, N = 14336, K = 4096: 22.6 -> 24.0 us); from
// four slices on it does (N = K = 4096: M = 128 21.0 -> 13.2 us, M = 256
// 21.2 -> 16.5 us; M = 128, N = 1024, K = 16384 in 13.2 us, M = N = 256,
// K = 8192 in 10.0 us). From K = 8192 on, two slices over 65..128 tiles do
// earn it back. Sized for the 256 CUs of an MI355X rather than the device at
// hand, so launch, scratch sizing and the check agree. 1: no split.
constexpr int64_t kSplitCus = 256;
template <int BM, int BN>
int mfma_k_split(const Problem &r) {
  if (r.batch != 1 || r.K < 1024 || r.N % 16) return 1;
  const int64_t tiles = (r.M + BM - 1) / BM * ((r.N + BN - 1) / BN);
  if (tiles * 4 > kSplitCus) return tiles * 2 <= kSplitCus && r.K >= 8192 && r.K % 256 == 0 ? 2 : 1;
  int ks = 1;
  while (ks < 16 && 2 * ks * tiles <= kSplitCus) ks *= 2;
  while (ks > 1 && (r.K % (128 * ks) || r.K / ks < 512)) ks /= 2;
  return ks;
}

// Whether the persistent 256x256 kernels take a row-major problem: K in whole
// 64-deep slices and M, N at least one tile (N is a multiple of 16 on every
// vector path). A last tile row or column past M or N is moved back to end
// there; the rows and columns it shares with its neighbour are stored by the
// neighbour alone (their EDGE instantiations), so every element of C is
// written once and in-place C = C + A.B adds D once.
bool persistent_fits(const Problem &r) {
  return r.K > 0 && r.K % 64 == 0 && r.M >= 256 && r.N >= 256;
}

// Rows of a row-major 256x256 problem (after the fold) that run on the
// persistent kernel before the rest run on 128x128 tiles: the whole 256-row
// tiles, when N is whole tiles and the last, partial tile row would add a
// round of tiles on a 256-CU chip (M = 1100, N = 14336, K = 4096: 224 + 56
// tiles; 114 us as 280 tiles, 78 us split). 0: one launch.
int64_t mfma_split_rows(const Problem &r) {
  if (r.M < 256 || r.M % 256 == 0 || r.N % 256 || r.K == 0 || r.K % 64) return 0;
  const int64_t row_tiles = r.N / 256 * r.batch, full = r.M / 256 * row_tiles;
  const bool more_rounds = (full + row_tiles + kSplitCus - 1) / kSplitCus > (full + kSplitCus - 1) / kSplitCus;
  return more_rounds ? r.M / 256 * 256 : 0;
}

// The same for columns: the whole 256-column tiles first, when M is whole
// tiles and the last, partial tile column would add a round of tiles
// (M = 8192, N = 8208: 1024 + 32 tiles). 0: one launch.
int64_t mfma_split_cols(const Problem &r) {
  if (r.N < 256 || r.N % 256 == 0 || r.M % 256 || r.K == 0 || r.K % 64) return 0;
  const int64_t col_tiles = r.M / 256 * r.batch, full = r.N / 256 * col_tiles;
  const bool more_rounds = (full + col_tiles + kSplitCus - 1) / kSplitCus > (full + kSplitCus - 1) / kSplitCus;
  return more_rounds ? r.N / 256 * 256 : 0;
}

// Columns [c0, N) of a problem, in every batch (c0 a multiple of 256, so B,
// C and D keep their alignment).
Problem cols_from(const Problem &r, int64_t c0) {
  Problem g = r;
  g.B = r.B + c0;
  g.C = r.C + c0;
  g.D = r.D ? r.D + c0 : nullptr;
  g.N = r.N - c0;
  return g;
}

// Rows [r0, M) of a problem, in every batch.
Problem rows_from(const Problem &r, int64_t r0) {
  Problem g = r;
  g.A = r.A + r0 * r.lda;
  g.C = r.C + r0 * r.ldc;
  g.D = r.D ? r.D + r0 * r.ldd : nullptr;
  g.M = r.M - r0;
  return g;
}

// The K split vt_gemm_i8 launches for an MFMA variant (1 for the others).
// The mfma_128x128 variant with row-major B runs 64x128 tiles (and the K
// split those tiles call for) when that gives at most one workgroup per CU
// over at most 2048 of K, or 1024 per slice when K is split: twice the 128x128
// workgroups, or fewer K slices (often none, and no reduction launch), with
// half the A rows and C per workgroup. On grids that small the workgroups'
// loads are the critical path. HIP graph per launch, interleaved on one box,
// 128x128 against 64x128 tiles: 256^3 + D 5.31 -> 4.10 us, 512^2 x 512
// 5.27 -> 4.37, 300 x 208 x 160 6.14 -> 4.79, 1024^2 x 512 5.78 -> 5.13,
// 1024^3 12.4 (two K slices) -> 6.2 (none), 1024^2 x 2048 15.6 (four) -> 11.5
// (none), 256 x 4096 x 2048 13.3 -> 11.6, 256 x 2048 x 4096 13.6 -> 11.8,
// 128 x 4096 x 4096 13.5 (eight slices) -> 12.9 (four), and the remainders
// of split 256x256 launches 3-5 %. Outside the rule 64-row tiles lost:
// 2048^2 x 512 (512 workgroups) 9 %, 1536^2 x 1024 (288) 12 %,
// 256 x 4096 x 4096 (K 4096 unsplit) 25 %, 128 x 4096 x 8192 (four slices of
// 2048 against eight of 1024) 7 %.
constexpr int64_t kHalfTileMaxWgs = 256, kHalfTileMaxK = 2048, kHalfTileMaxSliceK = 1024;

// r: the folded problem (mfma_fold).
bool mfma_half_rows(const Problem &r) {
  const int ks = mfma_k_split<64, 128>(r);
  const int64_t wgs = (r.M + 63) / 64 * ((r.N + 127) / 128) * r.batch * ks;
  return wgs <= kHalfTileMaxWgs && r.K / ks <= (ks > 1 ? kHalfTileMaxSliceK : kHalfTileMaxK);
}

// Within that rule, 64x64 tiles (one 32x32 block per wave) when they too,
// with their own K split, give at most one workgroup per CU over at most 2048
// of K (1024 per slice when split): half of each workgroup's B panel and C
// again. Interleaved on one box, HIP graph per launch, 64x128 against 64x64
// tiles: 256^3 + D (config 2) 4.14-4.15 -> 3.36-3.37 us, 512^3 4.35 -> 3.61,
// 300 x 208 x 160 4.80-4.85 -> 3.75, 192^3 4.77 -> 3.72, 128^3 + D 3.17 ->
// 2.64, 1024^2 x 512 4.62 -> 4.07, 1024^3 6.20 -> 5.43, 1024^2 x 2048 11.63
// -> 10.96, 512^2 x 2048 + D 8.6-8.9 -> 8.08, 256 x 4096 x 2048 11.6 ->
// 11.06, 128 x 4096 x 1152 6.28 -> 5.31, 256^2 x 8192 + D 8.9 -> 8.5,
// 512^2 x 256 3.61 -> 3.00, 256 x 512 x 1024 + D 7.23 -> 6.56,
// 256 x 1024 x 4096 (eight K slices -> four) 10.87 -> 9.74, 128 x 256 x 8192
// 8.32 -> 7.62, 96 x 2048 x 2048 8.79 -> 8.0, 100 x 208 x 2048 + D 7.36 ->
// 6.42; the shapes outside the rule (128 x 4096 x 4096, 96 x 4096 x 4096,
// 128 x 1024 x 16384) measured the same in both builds.
bool mfma_quarter_tiles(const Problem &r) {
  if (!mfma_half_rows(r)) return false;
  const int ks = mfma_k_split<64, 64>(r);
  const int64_t wgs = (r.M + 63) / 64 * ((r.N + 63) / 64) * r.batch * ks;
  return wgs <= kHalfTileMaxWgs && r.K / ks <= (ks > 1 ? kHalfTileMaxSliceK : kHalfTileMaxK);
}

// K slices of an mfma_128x128 launch with row-major B (r folded).
int mfma128_split(const Problem &r) {
  if (mfma_quarter_tiles(r)) return mfma_k_split<64, 64>(r);
  return mfma_half_rows(r) ? mfma_k_split<64, 128>(r) : mfma_k_split<128, 128>(r);
}

int mfma_split_for(const Problem &q, int32_t variant) {
  const Problem r = mfma_fold(q);
  switch (variant) {
    case VT_VARIANT_MFMA_256x256: return mfma_k_split<256, 256>(r);
    case VT_VARIANT_MFMA_128x128: return mfma128_split(r);
    case VT_VARIANT_MFMA_256x128: return mfma_k_split<256, 128>(r);
    default: return 1;
  }
}

// Packed B on 128x128 MFMA tiles: lane offsets from a tile's base within 32
// bits (A: 256 rows of lda; packed B: 8 column blocks of kbt 1 KB tiles).
bool packed_tiles_fit(const Problem &q) {
  return (__int128)256 * q.lda < (1ll << 32) - 4096 &&
         (__int128)8 * 1024 * ((q.K + 63) / 64) < (1ll << 32) - 4096;
}

template <int BM, int BN, bool PACKED = false>
int launch_mfma_tiles(const Problem &r, hipStream_t stream, int num_cus);

int launch_mfma128(const Problem &q, Scratch &scr);

template <int BM, int BN, bool PACKED = false>
int launch_mfma(const Problem &q, Scratch &scr) {
  const Problem r = mfma_fold(q);
  if (PACKED ? !packed_tiles_fit(r) : !mfma_addressable(r))
    return fail(VT_EUNSUPPORTED,
                "MFMA variants need 256*lda and 64*ldb below 2^32 (lda=%lld ldb=%lld)",
                (long long)r.lda, (long long)r.ldb);
  hipStream_t stream = (hipStream_t)scr.stream;
  const int num_cus = scr.st->num_cus;
  const int ks = mfma_k_split<BM, BN>(r);
  if constexpr (!PACKED && BM == 256 && BN == 256) {
    if (const int64_t rows = ks == 1 ? mfma_split_rows(r) : 0) {
      Problem top = r;
      top.M = rows;
      if (int rc = launch_mfma_tiles<BM, BN, PACKED>(top, stream, num_cus)) return rc;
      return launch_mfma128(rows_from(r, rows), scr);
    }
    if (const int64_t cols = ks == 1 ? mfma_split_cols(r) : 0) {
      Problem left = r;
      left.N = cols;
      if (int rc = launch_mfma_tiles<BM, BN, PACKED>(left, stream, num_cus)) return rc;
      return launch_mfma128(cols_from(r, cols), scr);
    }
  }
  if (ks == 1) return launch_mfma_tiles<BM, BN, PACKED>(r, stream, num_cus);
  // K slices as batches: slice i reads A columns and B rows [i*kc, (i+1)*kc)
  // and writes its partial sums to slice i of the workspace.
  void *w = nullptr;
  int rc = scr.take(kPartials, (size_t)ks * r.M * r.N * sizeof(int32_t), &w);
  if (rc) return rc;
  const int64_t kc = r.K / ks;
  Problem sl = r;
  sl.K = kc;
  sl.batch = ks;
  sl.sa = kc;
  sl.sb = PACKED ? kc / 64 * 1024 : kc * r.ldb;   // packed: the slice's first 64-row block
  sl.D = nullptr;
  sl.sd = 0;
  sl.C = (int32_t *)w;
  sl.ldc = r.N;
  sl.sc = r.M * r.N;
  rc = launch_mfma_tiles<BM, BN, PACKED>(sl, stream, num_cus);
  if (rc) return rc;
  ReduceArgs ra;
  ra.ws = (const int32_t *)w; ra.D = r.D; ra.C = r.C;
  ra.ldd = r.ldd; ra.ldc = r.ldc; ra.sd = 0; ra.sc = 0;
  ra.M = (int)r.M; ra.N = (int)r.N; ra.k_split = ks;
  return launch_reduce(ra, 1, stream);
}

template <int BM, int BN, bool PACKED>
int launch_mfma_tiles(const Problem &r, hipStream_t stream, int num_cus) {
  GemmArgs a;
  a.A = r.A; a.B = r.B; a.D = r.D; a.C = r.C;
  a.lda = r.lda; a.ldb = r.ldb; a.ldd = r.ldd; a.ldc = r.ldc;
  a.sa = r.sa; a.sb = r.sb; a.sd = r.sd; a.sc = r.sc;
  a.M = (int)r.M; a.N = (int)r.N; a.K = (int)r.K;
  a.tiles_m = (int)((r.M + BM - 1) / BM);
  a.tiles_n = (int)((r.N + BN - 1) / BN);
  a.group_m = 4;
  const int64_t blocks = (int64_t)a.tiles_m * a.tiles_n * r.batch;
  if (blocks > 0x7fffffff) return fail(VT_EUNSUPPORTED, "grid of %lld tiles too large", (long long)blocks);
  const bool has_d = r.D != nullptr;
  dim3 grid((unsigned)blocks), block(256);
  a.batch_count = (int)r.batch;
  if (!PACKED && BM == 256 && BN == 256 && persistent_fits(r)) {
    // Persistent: one workgroup per CU (the kernel's LDS allows no more).
    const int64_t g = blocks < num_cus ? blocks : num_cus;
    dim3 pgrid((unsigned)g);
    const bool edge = r.M % BM || r.N % BN;
    if (use_dma16(r)) {
      if (edge && has_d) hipLaunchKernelGGL((gemm_dma16_kernel<true, false, true>), pgrid, dim3(256), 0, stream, a);
      else if (edge) hipLaunchKernelGGL((gemm_dma16_kernel<false, false, true>), pgrid, dim3(256), 0, stream, a);
      else if (has_d) hipLaunchKernelGGL((gemm_dma16_kernel<true, false>), pgrid, dim3(256), 0, stream, a);
      else hipLaunchKernelGGL((gemm_dma16_kernel<false, false>), pgrid, dim3(256), 0, stream, a);
    } else if (edge && has_d) {
      hipLaunchKernelGGL((gemm_dma_kernel<kDmaWaves, true, false, true>), pgrid, dim3(64 * kDmaWaves), 0, stream, a);
    } else if (edge) {
      hipLaunchKernelGGL((gemm_dma_kernel<kDmaWaves, false, false, true>), pgrid, dim3(64 * kDmaWaves), 0, stream, a);
    } else if (has_d) {
      hipLaunchKernelGGL((gemm_dma_kernel<kDmaWaves, true>), pgrid, dim3(64 * kDmaWaves), 0, stream, a);
    } else {
      hipLaunchKernelGGL((gemm_dma_kernel<kDmaWaves, false>), pgrid, dim3(64 * kDmaWaves), 0, stream, a);
    }
    VT_HIP_CHECK(hipGetLastError());
    return VT_OK;
  }
  if (!PACKED && BM == 256 && BN == 128 && dma16_128_fits(r)) {
    const int64_t g = blocks < num_cus ? blocks : num_cus;
    const dim3 pgrid((unsigned)g);
    const bool edge = r.M % BM || r.N % BN;
    if (edge && has_d) hipLaunchKernelGGL((gemm_dma16_kernel<true, false, true, 128>), pgrid, dim3(256), 0, stream, a);
    else if (edge) hipLaunchKernelGGL((gemm_dma16_kernel<false, false, true, 128>), pgrid, dim3(256), 0, stream, a);
    else if (has_d) hipLaunchKernelGGL((gemm_dma16_kernel<true, false, false, 128>), pgrid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((gemm_dma16_kernel<false, false, false, 128>), pgrid, dim3(256), 0, stream, a);
    VT_HIP_CHECK(hipGetLastError());
    return VT_OK;
  }
  const int edge = (r.K % 128) ? 2 : ((r.M % BM) || (r.N % BN)) ? 1 : 0;
  const bool short_k = r.K <= 128;
  const bool early_d = blocks <= num_cus;   // one workgroup per CU: occupancy costs nothing
  if (edge == 2) {
    if (has_d) launch_mfma_kernel<BM, BN, 2, true, PACKED>(short_k, early_d, grid, block, stream, a);
    else launch_mfma_kernel<BM, BN, 2, false, PACKED>(short_k, early_d, grid, block, stream, a);
  } else if (edge == 1) {
    if (has_d) launch_mfma_kernel<BM, BN, 1, true, PACKED>(short_k, early_d, grid, block, stream, a);
    else launch_mfma_kernel<BM, BN, 1, false, PACKED>(short_k, early_d, grid, block, stream, a);
  } else {
    if (has_d) launch_mfma_kernel<BM, BN, 0, true, PACKED>(short_k, early_d, grid, block, stream, a);
    else launch_mfma_kernel<BM, BN, 0, false, PACKED>(short_k, early_d, grid, block, stream, a);
  }
  VT_HIP_CHECK(hipGetLastError());
  return VT_OK;
}

// The mfma_128x128 variant with row-major B: 64x64, 64x128 or 128x128 tiles
// (mfma_quarter_tiles, mfma_half_rows).
int launch_mfma128(const Problem &q, Scratch &scr) {
  if (mfma_quarter_tiles(mfma_fold(q))) return launch_mfma<64, 64>(q, scr);
  if (mfma_half_rows(mfma_fold(q))) return launch_mfma<64, 128>(q, scr);
  return launch_mfma<128, 128>(q, scr);
}

// K slices of the skinny kernel: rows per slice (a multiple of the pipeline
// length, shrunk until the A part fits in LDS), the split count that gives,
// and the dynamic LDS bytes.
struct SkinnyGeom {
  int64_t chunk, lds;
  int ks;
};

template <int NB, int WAVES, int U>
SkinnyGeom skinny_geometry(const Problem &q, int k_split) {
  constexpr int R = WAVES * 1024 / NB;           // rows per stage
  constexpr int64_t kAlign = (int64_t)R * U;     // rows per unrolled pipeline
  constexpr int64_t kStageLds = 2 * (int64_t)R * NB;
  const int64_t a_rows = 16 * (int64_t)skinny_row_blocks(q.M);   // LDS rows of the A slice
  if (k_split <= 0) k_split = choose_k_split(q.N, q.K, q.batch);
  int64_t chunk = (q.K + k_split - 1) / k_split;
  chunk = (chunk + kAlign - 1) / kAlign * kAlign;
  int64_t lds = a_rows * skinny_a_stride((int)chunk) + kStageLds;
  if (lds > kMaxSkinnyLds) {
    // skinny_a_stride adds at most 48 bytes to a row
    chunk = ((kMaxSkinnyLds - kStageLds) / a_rows - 48) / kAlign * kAlign;
    lds = a_rows * skinny_a_stride((int)chunk) + kStageLds;
  }
  return SkinnyGeom{chunk, lds, (int)((q.K + chunk - 1) / chunk)};
}

template <int NB, int WAVES, int U, int MB, bool FIN = false>
void launch_skinny_kernel(bool has_d, dim3 grid, dim3 block, size_t lds, hipStream_t s,
                          const SkinnyArgs &a) {
  if (has_d) hipLaunchKernelGGL((skinny_kernel<NB, WAVES, U, MB, true, FIN>), grid, block, lds, s, a);
  else hipLaunchKernelGGL((skinny_kernel<NB, WAVES, U, MB, false, FIN>), grid, block, lds, s, a);
}

// Field width of the finishing word for k_split slices of chunk rows (the bit
// length of the largest sum of biased partials), or 0 when two such fields
// leave no room for the count (or there is no split).
int skinny_fin_bits(int ks, int64_t chunk) {
  if (ks < 2 || chunk < 1) return 0;
  const uint64_t top = (uint64_t)ks * (uint64_t)chunk * (uint64_t)kFinSpanPerRow;
  const int bits = 64 - __builtin_clzll(top);
  const int count_bits = 64 - __builtin_clzll((uint64_t)(ks - 1));
  return 2 * bits + count_bits <= 64 ? bits : 0;
}

// Whether a K-split skinny launch finishes its sums in the kernel: few rows,
// a finishing-word count that fits, and a per-stream workspace (the fixed
// scratch of vt_gemm_i8_noalloc is not kept zero, so those calls take the
// second launch).
bool skinny_finishes(int64_t M, int ks, int64_t chunk, const Scratch &scr) {
  return ks > 1 && M <= kSkinnyFinMaxM && !scr.fixed && skinny_fin_bits(ks, chunk) > 0;
}

template <int NB, int WAVES, int U>
int launch_skinny_cfg(const Problem &q, int k_split, Scratch &scr) {
  if (q.M > kSkinnyMaxM)
    return fail(VT_EUNSUPPORTED, "skinny variant needs M <= %d (M=%lld)", kSkinnyMaxM, (long long)q.M);
  const SkinnyGeom geo = skinny_geometry<NB, WAVES, U>(q, k_split);
  const int64_t chunk = geo.chunk, lds = geo.lds;
  const int ks = geo.ks;
  SkinnyArgs a;
  a.A = q.A; a.B = q.B; a.D = q.D; a.C = q.C;
  a.lda = q.lda; a.ldb = q.ldb; a.ldd = q.ldd; a.ldc = q.ldc;
  a.sa = q.sa; a.sb = q.sb; a.sd = q.sd; a.sc = q.sc;
  a.M = (int)q.M; a.N = (int)q.N; a.K = (int)q.K;
  a.tiles_n = (int)((q.N + NB - 1) / NB);
  a.k_split = ks;
  a.k_chunk = (int)chunk;
  a.ws = nullptr;
  a.fin = nullptr;
  a.fin_bits = 0;
  if ((int64_t)a.tiles_n * ks > 0x7fffffff || q.batch > 65535)
    return fail(VT_EUNSUPPORTED, "skinny grid too large");
  const bool fin = skinny_finishes(q.M, ks, chunk, scr);
  if (fin) {
    void *w = nullptr;
    int rc = scr.take(kFinWords, (size_t)q.batch * ((q.M + 1) / 2) * q.N * sizeof(uint64_t), &w);
    if (rc) return rc;
    a.fin = (uint64_t *)w;
    a.fin_bits = skinny_fin_bits(ks, chunk);
  } else if (ks > 1) {
    void *w = nullptr;
    const size_t pbytes = (size_t)q.batch * ks * q.M * q.N * sizeof(int32_t);
    int rc = scr.take(kPartials, pbytes, &w);
    if (rc) return rc;
    a.ws = (int32_t *)w;
  }
  hipStream_t s = (hipStream_t)scr.stream;
  dim3 grid((unsigned)(a.tiles_n * ks), (unsigned)q.batch), block(64 * WAVES);
  // D is added by the kernel that completes a sum: this one without a K
  // split or when it finishes the slices itself, else the reduction.
  const bool d_in = q.D && (ks == 1 || fin);
  if (fin) {
    launch_skinny_kernel<NB, WAVES, U, 1, true>(d_in, grid, block, (size_t)lds, s, a);
    VT_HIP_CHECK(hipGetLastError());
    return VT_OK;
  }
  switch (skinny_row_blocks(q.M)) {
    case 1: launch_skinny_kernel<NB, WAVES, U, 1>(d_in, grid, block, (size_t)lds, s, a); break;
    case 2: launch_skinny_kernel<NB, WAVES, U, 2>(d_in, grid, block, (size_t)lds, s, a); break;
    default: launch_skinny_kernel<NB, WAVES, U, 4>(d_in, grid, block, (size_t)lds, s, a); break;
  }
  VT_HIP_CHECK(hipGetLastError());
  if (ks > 1) {
    ReduceArgs r;
    r.ws = a.ws; r.D = q.D; r.C = q.C;
    r.ldd = q.ldd; r.ldc = q.ldc; r.sd = q.sd; r.sc = q.sc;
    r.M = (int)q.M; r.N = (int)q.N; r.k_split = ks;
    const int rc = launch_reduce(r, q.batch, s);
    if (rc) return rc;
  }
  return VT_OK;
}

int launch_skinny(const Problem &q, int k_split, Scratch &scr) {
  return launch_skinny_cfg<kSkinnyNB, kSkinnyWaves, kSkinnyU>(q, k_split, scr);
}

// Packed-B decode configuration: 4 column blocks (64 columns) per workgroup,
// 8 waves, 2 row blocks of loads ahead. For N = 14336 that is 224 workgroups
// streaming 256 KiB each.
constexpr int kPackedNBW = 4, kPackedWaves = 8, kPackedS = 2;

int64_t packed_kbt(int64_t K) { return (K + 63) / 64; }

// Half blocks per column group. Whole groups of NBW blocks when they alone
// give 192 or more workgroups (N = 14336: 224 groups). Below that, groups as
// small as needed for one per CU, at half-block granularity, instead of a K
// split and a second kernel: measured at K = 4096, N = 1024 .. 8192 run 16-22 %
// faster that way. At N = 14336, 256 groups of 3.5 blocks ran 3 % slower than
// 224 groups of 4, so larger N keeps whole groups.
int packed_hpw(int64_t N, int64_t batch, int num_cus) {
  const int64_t nbt = N / 16;
  if ((nbt + kPackedNBW - 1) / kPackedNBW * batch >= 192) return 2 * kPackedNBW;
  int64_t h = (2 * nbt * batch + num_cus - 1) / num_cus;
  if (h < 1) h = 1;
  if (h > 2 * kPackedNBW) h = 2 * kPackedNBW;
  return (int)h;
}

// Workgroups along K for the packed kernel, given the column groups of all
// batches: 1 when those alone give most CUs a workgroup, else enough K slices
// for ~224 workgroups, each slice at least one row block per wave.
int packed_k_split(int64_t groups, int64_t K) {
  if (groups >= 192) return 1;
  int64_t ks = (224 + groups - 1) / groups;
  const int64_t max_by_k = (packed_kbt(K) + kPackedWaves - 1) / kPackedWaves;
  if (ks > max_by_k) ks = max_by_k;
  if (ks < 1) ks = 1;
  if (ks > 64) ks = 64;
  return (int)ks;
}

// Whether the rows of a packed-B GEMM in whole 256-row tiles can run on the
// 256x256 DMA kernel: N in whole 256-column tiles, K in whole 64-deep slices,
// and every lane offset from a tile's base within 32 bits (A: 256 rows of
// lda; packed B: 16 column blocks of kbt 1 KB tiles).
bool packed_dma_fits(const Problem &q) {
  return q.M >= 256 && q.N % 256 == 0 && q.K % 64 == 0 && q.K > 0 &&
         256 * q.lda < (1ll << 32) - 4096 && 16 * 1024 * packed_kbt(q.K) < (1ll << 32) - 4096;
}

// Whole 256-row tiles of a packed-B GEMM go to the persistent 256x256 DMA
// kernel when there are at least this many of them (over all batches); fewer
// run faster as 128x128 tiles (N = 14336, K = 4096: 512 rows, 112 tiles,
// 46.6 us on the DMA kernel against 43.2 us; 768 rows, 168 tiles, 55.1 us
// against 63.4 us).
constexpr int64_t kPackedDmaMinTiles = 128;

// Rows of a packed-B GEMM that run on the persistent 256x256 DMA kernel: all
// of them when its partial last tile row (moved back to end at M, its stores
// masked to the rows no other tile writes) adds no round of tiles on a
// 256-CU chip, else the whole 256-row tiles; 0 when fewer than
// kPackedDmaMinTiles whole tiles exist.
int64_t packed_dma_rows(const Problem &q) {
  if (!packed_dma_fits(q)) return 0;
  const int64_t row_tiles = q.N / 256 * q.batch, full = q.M / 256 * row_tiles;
  if (full < kPackedDmaMinTiles) return 0;
  if (q.M % 256 == 0) return q.M;
  const bool more_rounds =
      (full + row_tiles + kSplitCus - 1) / kSplitCus > (full + kSplitCus - 1) / kSplitCus;
  return more_rounds ? q.M / 256 * 256 : q.M;
}

// Rows [0, rows) of a packed-B GEMM (rows from packed_dma_rows) on the
// persistent 256x256 DMA kernel, every batch in one launch.
int launch_packed_dma(const Problem &q, int64_t rows, hipStream_t stream, int num_cus) {
  GemmArgs a;
  a.A = q.A; a.B = q.B; a.D = q.D; a.C = q.C;
  a.lda = q.lda; a.ldb = packed_kbt(q.K); a.ldd = q.ldd; a.ldc = q.ldc;
  a.sa = q.sa; a.sb = q.sb; a.sd = q.sd; a.sc = q.sc;
  a.M = (int)rows; a.N = (int)q.N; a.K = (int)q.K;
  a.tiles_m = (a.M + 255) / 256;
  a.tiles_n = a.N / 256;
  a.group_m = 4;
  a.batch_count = (int)q.batch;
  const int64_t blocks = (int64_t)a.tiles_m * a.tiles_n * q.batch;
  if (blocks > 0x7fffffff) return fail(VT_EUNSUPPORTED, "grid of %lld tiles too large", (long long)blocks);
  dim3 pgrid((unsigned)(blocks < num_cus ? blocks : num_cus));
  const bool edge = rows % 256 != 0;
  if (use_dma16(q)) {
    if (edge && q.D) hipLaunchKernelGGL((gemm_dma16_kernel<true, true, true>), pgrid, dim3(256), 0, stream, a);
    else if (edge) hipLaunchKernelGGL((gemm_dma16_kernel<false, true, true>), pgrid, dim3(256), 0, stream, a);
    else if (q.D) hipLaunchKernelGGL((gemm_dma16_kernel<true, true>), pgrid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((gemm_dma16_kernel<false, true>), pgrid, dim3(256), 0, stream, a);
  } else if (edge && q.D) {
    hipLaunchKernelGGL((gemm_dma_kernel<kDmaWaves, true, true, true>), pgrid, dim3(64 * kDmaWaves), 0, stream, a);
  } else if (edge) {
    hipLaunchKernelGGL((gemm_dma_kernel<kDmaWaves, false, true, true>), pgrid, dim3(64 * kDmaWaves), 0, stream, a);
  } else if (q.D) {
    hipLaunchKernelGGL((gemm_dma_kernel<kDmaWaves, true, true>), pgrid, dim3(64 * kDmaWaves), 0, stream, a);
  } else {
    hipLaunchKernelGGL((gemm_dma_kernel<kDmaWaves, false, true>), pgrid, dim3(64 * kDmaWaves), 0, stream, a);
  }
  VT_HIP_CHECK(hipGetLastError());
  return VT_OK;
}

// A packed-B GEMM runs whole on the 256x128 form of the persistent kernel
// when the 256x256 kernel does not take it (packed_dma_rows == 0), K >= 1024
// and there are more than 128 but at most 256 tiles of 256x128 (over all
// batches), as for row-major B; it needs M >= 256 (a partial last tile row
// moved back), N in whole 128-column tiles, K in whole 256-deep groups,
// 16-byte C and D rows, and every lane offset from a tile's base within 32
// bits (A: 256 rows of lda; packed B: 8 column blocks of kbt 1 KB tiles).
// Against the 128x128 packed tiles it replaced there (HIP graphs, one box):
// 1536 x 4096 x 4096 30.9 us against 36.4, 1536 x 4096 x 8192 55.1 against
// 67.7, 512 x 14336 x 4096 32.4 against 40.5, 2000 x 4096 x 4096 35.8
// against 43.6; at 128 tiles or fewer it lost (1024 x 4096 x 4096 28.1
// against 25.4, 300 x 4096 x 4096 27.1 against 20.7).
bool packed_dma128_fits(const Problem &q) {
  if (!(q.M >= 256 && q.N % 128 == 0 && q.K % 256 == 0 && q.K >= 1024 &&
        256 * q.lda < (1ll << 32) - 4096 && 8 * 1024 * packed_kbt(q.K) < (1ll << 32) - 4096 &&
        q.ldc < (1ll << 28) && (!q.D || q.ldd < (1ll << 28)) && use_dma16(q)))
    return false;
  const int64_t tiles = (q.M + 255) / 256 * (q.N / 128) * q.batch;
  return tiles > 128 && tiles <= 256;
}

int launch_packed_dma128(const Problem &q, hipStream_t stream, int num_cus) {
  GemmArgs a;
  a.A = q.A; a.B = q.B; a.D = q.D; a.C = q.C;
  a.lda = q.lda; a.ldb = packed_kbt(q.K); a.ldd = q.ldd; a.ldc = q.ldc;
  a.sa = q.sa; a.sb = q.sb; a.sd = q.sd; a.sc = q.sc;
  a.M = (int)q.M; a.N = (int)q.N; a.K = (int)q.K;
  a.tiles_m = (a.M + 255) / 256;
  a.tiles_n = a.N / 128;
  a.group_m = 4;
  a.batch_count = (int)q.batch;
  const int64_t blocks = (int64_t)a.tiles_m * a.tiles_n * q.batch;
  if (blocks > 0x7fffffff) return fail(VT_EUNSUPPORTED, "grid of %lld tiles too large", (long long)blocks);
  const dim3 pgrid((unsigned)(blocks < num_cus ? blocks : num_cus));
  const bool edge = q.M % 256 != 0;
  if (edge && q.D) hipLaunchKernelGGL((gemm_dma16_kernel<true, true, true, 128>), pgrid, dim3(256), 0, stream, a);
  else if (edge) hipLaunchKernelGGL((gemm_dma16_kernel<false, true, true, 128>), pgrid, dim3(256), 0, stream, a);
  else if (q.D) hipLaunchKernelGGL((gemm_dma16_kernel<true, true, false, 128>), pgrid, dim3(256), 0, stream, a);
  else hipLaunchKernelGGL((gemm_dma16_kernel<false, true, false, 128>), pgrid, dim3(256), 0, stream, a);
  VT_HIP_CHECK(hipGetLastError());
  return VT_OK;
}

template <int MB, bool FIN = false>
void launch_packed_kernel(bool d_in, bool masked, dim3 grid, dim3 block, hipStream_t s,
                          const PackedArgs &a) {
  if (d_in && masked)
    hipLaunchKernelGGL((packed_skinny_kernel<kPackedNBW, kPackedWaves, kPackedS, MB, true, true, FIN>), grid, block, 0, s, a);
  else if (d_in)
    hipLaunchKernelGGL((packed_skinny_kernel<kPackedNBW, kPackedWaves, kPackedS, MB, true, false, FIN>), grid, block, 0, s, a);
  else if (masked)
    hipLaunchKernelGGL((packed_skinny_kernel<kPackedNBW, kPackedWaves, kPackedS, MB, false, true, FIN>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((packed_skinny_kernel<kPackedNBW, kPackedWaves, kPackedS, MB, false, false, FIN>), grid, block, 0, s, a);
}

// One launch (plus the partial-sum reduction when K is split) over at most
// kSkinnyMaxM (64) rows of A / C / D: 1, 2 or 4 row blocks of 16.
int launch_packed_rows(const Problem &q, int k_split, Scratch &scr) {
  PackedArgs a;
  a.A = q.A; a.Bp = q.B; a.D = q.D; a.C = q.C;
  a.lda = q.lda; a.ldd = q.ldd; a.ldc = q.ldc;
  a.sa = q.sa; a.sbp = q.sb; a.sd = q.sd; a.sc = q.sc;
  a.M = (int)q.M; a.N = (int)q.N; a.K = (int)q.K;
  a.kbt = (int)packed_kbt(q.K);
  a.hpw = packed_hpw(q.N, q.batch, scr.st->num_cus);
  a.groups = (int)((2 * (q.N / 16) + a.hpw - 1) / a.hpw);
  const int ks0 = k_split > 0 ? k_split : packed_k_split((int64_t)a.groups * q.batch, q.K);
  a.kb_per_split = (a.kbt + ks0 - 1) / ks0;
  a.k_split = (a.kbt + a.kb_per_split - 1) / a.kb_per_split;
  a.ws = nullptr;
  a.fin = nullptr;
  a.fin_bits = 0;
  if ((int64_t)a.groups * a.k_split > 0x7fffffff || q.batch > 65535)
    return fail(VT_EUNSUPPORTED, "packed grid too large");
  // The K slices finish in the kernel on the skinny kernel's terms (few
  // rows, a count that fits beside the fields, a per-stream workspace).
  const bool fin = skinny_finishes(q.M, a.k_split, (int64_t)a.kb_per_split * 64, scr);
  if (fin) {
    void *w = nullptr;
    int rc = scr.take(kFinWords, (size_t)q.batch * ((q.M + 1) / 2) * q.N * sizeof(uint64_t), &w);
    if (rc) return rc;
    a.fin = (uint64_t *)w;
    a.fin_bits = skinny_fin_bits(a.k_split, (int64_t)a.kb_per_split * 64);
  } else if (a.k_split > 1) {
    void *w = nullptr;
    const size_t pbytes = (size_t)q.batch * a.k_split * q.M * q.N * sizeof(int32_t);
    int rc = scr.take(kPartials, pbytes, &w);
    if (rc) return rc;
    a.ws = (int32_t *)w;
  }
  hipStream_t s = (hipStream_t)scr.stream;
  dim3 grid((unsigned)(a.groups * a.k_split), (unsigned)q.batch), block(64 * kPackedWaves);
  const bool d_in = q.D && (a.k_split == 1 || fin), masked = a.hpw != 2 * kPackedNBW;
  if (fin) {
    launch_packed_kernel<1, true>(d_in, masked, grid, block, s, a);
    VT_HIP_CHECK(hipGetLastError());
    return VT_OK;
  }
  switch (skinny_row_blocks(q.M)) {
    case 1: launch_packed_kernel<1>(d_in, masked, grid, block, s, a); break;
    case 2: launch_packed_kernel<2>(d_in, masked, grid, block, s, a); break;
    default: launch_packed_kernel<4>(d_in, masked, grid, block, s, a); break;
  }
  VT_HIP_CHECK(hipGetLastError());
  if (a.k_split > 1) {
    ReduceArgs r;
    r.ws = a.ws; r.D = q.D; r.C = q.C;
    r.ldd = q.ldd; r.ldc = q.ldc; r.sd = q.sd; r.sc = q.sc;
    r.M = (int)q.M; r.N = (int)q.N; r.k_split = a.k_split;
    const int rc = launch_reduce(r, q.batch, s);
    if (rc) return rc;
  }
  return VT_OK;
}

// ---------------------------------------------------------------------------
// Padded path: any shape through the vector kernels
// ---------------------------------------------------------------------------

// Zero-padded int8 copy: dst[b][r][c] (r < rows_p, c < cols_p, cols_p % 16 == 0)
// is src[b*ss + r*ld + c] where r < rows and c < cols, else 0. One thread
// writes 16 bytes. The source may have any alignment and stride: interior
// chunks are read as aligned dwords that never leave the row, the row's
// edges bytewise. A and B are copied by one launch: blockIdx.z picks the
// operand, and blocks past that operand's grid or batch count exit.
struct PadArgs {
  const int8_t *src;
  int8_t *dst;
  int64_t ld, ss, sd;
  int64_t rows, cols, rows_p, cols_p;
  int64_t batches;
};

__global__ __launch_bounds__(256) void pad_i8_kernel(PadArgs pa, PadArgs pb) {
  const PadArgs p = blockIdx.z ? pb : pa;
  const int64_t chunks = p.cols_p / 16;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t b = blockIdx.y;
  if (i >= p.rows_p * chunks || b >= p.batches) return;
  // 32-bit division whenever the index fits (64-bit division is a long
  // software sequence)
  const int64_t r = p.rows_p * chunks <= 0xffffffffll ? (int64_t)((uint32_t)i / (uint32_t)chunks)
                                                      : i / chunks;
  const int64_t c0 = (i - r * chunks) * 16;
  v4i out = v4i{0, 0, 0, 0};
  if (r < p.rows) {
    const int8_t *s = p.src + b * p.ss + r * p.ld;
    if (c0 >= 4 && c0 + 20 <= p.cols) {
      // Interior chunk: five aligned dwords starting at most 3 bytes before
      // it cover its 16 bytes and stay inside this row; shift them into place.
      const uintptr_t at = (uintptr_t)(s + c0);
      const uint32_t *w = (const uint32_t *)(at & ~(uintptr_t)3);
      const uint32_t sh = (uint32_t)(at & 3) * 8;
      uint32_t d[5];
#pragma unroll
      for (int t = 0; t < 5; ++t) d[t] = w[t];
#pragma unroll
      for (int t = 0; t < 4; ++t)
        out[t] = (int)(sh ? (d[t] >> sh) | (d[t + 1] << (32 - sh)) : d[t]);
    } else {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        uint32_t word = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int64_t c = c0 + 4 * w + t;
          if (c < p.cols) word |= (uint32_t)(uint8_t)s[c] << (8 * t);
        }
        out[w] = (int)word;
      }
    }
  }
  *(v4i *)(p.dst + b * p.sd + r * p.cols_p + c0) = out;
}

// C[b][r][c] = src[b][r][c] (+ D[b][r][c]) for c < N: the padded product's
// valid columns, wrapping mod 2^32. Elementwise, so D may be C itself. One
// thread takes 4 columns: the source (workspace base, row pitch lds and
// batch stride ss all multiples of 16 bytes, lds >= N rounded up to 4) is
// read as one 16-byte load, C and D, of any alignment, per element.
struct UnpadArgs {
  const int32_t *src;
  const int32_t *D;
  int32_t *C;
  int64_t lds, ldd, ldc, ss, sd, sc;
  int64_t M, N;
};

template <bool HAS_D>
__global__ __launch_bounds__(256) void unpad_kernel(UnpadArgs p) {
  const int64_t quads = (p.N + 3) / 4;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= p.M * quads) return;
  const int64_t r = p.M * quads <= 0xffffffffll ? (int64_t)((uint32_t)i / (uint32_t)quads)
                                                : i / quads;
  const int64_t c0 = (i - r * quads) * 4, b = blockIdx.y;
  const v4i v = __builtin_nontemporal_load((const v4i *)(p.src + b * p.ss + r * p.lds + c0));
  const int32_t *d = HAS_D ? p.D + b * p.sd + r * p.ldd + c0 : nullptr;
  int32_t *c = p.C + b * p.sc + r * p.ldc + c0;
  int32_t dv[4] = {0, 0, 0, 0};
  if constexpr (HAS_D) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
      if (c0 + t < p.N) dv[t] = d[t];
  }
#pragma unroll
  for (int t = 0; t < 4; ++t)
    if (c0 + t < p.N) c[t] = add_wrap(v[t], dv[t]);
}

int launch_vector(const Problem &q, int32_t variant, int32_t k_split, Scratch &scr);

// A and B copied with K and N rounded up to 16 (zero columns of A meet zero
// rows of B, so the product is unchanged), multiplied by the kernel the
// vector path selects for the padded shape, valid columns copied out with D.
// An operand the vector kernels can already read (K, and N for B, multiples
// of 16, 16-byte aligned base, pitch and batch stride) is used in place, and
// when N is a multiple of 16 the product writes C (with D) directly.
// What the padded variant copies: K and N rounded up to 16, the A and B
// matrices (shared ones once) and, when N is not a multiple of 16, the
// padded product before its valid columns go out to C.
struct PaddedLayout {
  int64_t Kp, Np, bA, bB;
  bool copy_a, copy_b, copy_c;
  int64_t a_bytes, b_bytes, c_bytes;   // each rounded up to 256
};

PaddedLayout padded_layout(const Problem &q) {
  PaddedLayout L;
  L.Kp = (q.K + 15) / 16 * 16;
  L.Np = (q.N + 15) / 16 * 16;
  L.bA = (q.batch > 1 && q.sa == 0) ? 1 : q.batch;
  L.bB = (q.batch > 1 && q.sb == 0) ? 1 : q.batch;
  L.copy_a = L.Kp != q.K || q.lda % 16 || q.sa % 16 || !aligned16(q.A);
  L.copy_b = L.Kp != q.K || L.Np != q.N || q.ldb % 16 || q.sb % 16 || !aligned16(q.B);
  L.copy_c = L.Np != q.N;
  auto round256 = [](int64_t v) { return (v + 255) / 256 * 256; };
  L.a_bytes = L.copy_a ? round256(L.bA * q.M * L.Kp) : 0;
  L.b_bytes = L.copy_b ? round256(L.bB * L.Kp * L.Np) : 0;
  L.c_bytes = L.copy_c ? round256(q.batch * q.M * L.Np * 4) : 0;
  return L;
}

// The problem the vector kernels run for the padded variant, with the
// copies at Ap, Bp, Cp.
Problem padded_inner(const Problem &q, const PaddedLayout &L, int8_t *Ap, int8_t *Bp,
                     int32_t *Cp) {
  Problem g = q;
  g.N = L.Np;
  g.K = L.Kp;
  if (L.copy_a) {
    g.A = Ap;
    g.lda = L.Kp;
    g.sa = L.bA > 1 ? q.M * L.Kp : 0;
  }
  if (L.copy_b) {
    g.B = Bp;
    g.ldb = L.Np;
    g.sb = L.bB > 1 ? L.Kp * L.Np : 0;
  }
  if (L.copy_c) {
    g.C = Cp;
    g.ldc = L.Np;
    g.sc = q.M * L.Np;
    g.D = nullptr;
    g.ldd = L.Np;
    g.sd = 0;
  }
  return g;
}

// Bytes of scratch a launch of `variant` takes, counted as the fixed
// scratch buffer hands them out (each piece rounded up to 256).
int64_t scratch_need(const Problem &q, int32_t variant, int32_t k_split) {
  auto round256 = [](int64_t v) { return (v + 255) / 256 * 256; };
  if (variant == VT_VARIANT_SKINNY) {
    const SkinnyGeom geo = skinny_geometry<kSkinnyNB, kSkinnyWaves, kSkinnyU>(q, k_split);
    return geo.ks > 1 ? round256(q.batch * geo.ks * q.M * q.N * 4) : 0;
  }
  if (variant == VT_VARIANT_MFMA_256x256 || variant == VT_VARIANT_MFMA_128x128 ||
      variant == VT_VARIANT_MFMA_256x128) {
    const int ks = mfma_split_for(q, variant);
    const Problem r = mfma_fold(q);
    const bool split = variant == VT_VARIANT_MFMA_256x256 && ks == 1;
    const int64_t rows = split ? mfma_split_rows(r) : 0;
    const int64_t cols = split && !rows ? mfma_split_cols(r) : 0;
    if (rows || cols) {   // the rows or columns after the persistent kernel's, on 128x128 tiles
      const Problem g = mfma_fold(rows ? rows_from(r, rows) : cols_from(r, cols));
      const int ks2 = mfma128_split(g);
      return ks2 > 1 ? round256(ks2 * g.M * g.N * 4) : 0;
    }
    return ks > 1 ? round256(ks * r.M * r.N * 4) : 0;
  }
  if (variant != VT_VARIANT_PADDED || !padded_fits(q)) return 0;
  const PaddedLayout L = padded_layout(q);
  // distinct dummy bases, 16-byte aligned like the copies
  const Problem g = padded_inner(q, L, (int8_t *)(uintptr_t)256, (int8_t *)(uintptr_t)512,
                                 (int32_t *)(uintptr_t)768);
  int32_t v = 0, ks = 0;
  select_variant(g, true, &v, &ks);
  return L.a_bytes + L.b_bytes + L.c_bytes + scratch_need(g, v, ks);
}

int launch_padded(const Problem &q, Scratch &scr) {
  if (!padded_fits(q))
    return fail(VT_EUNSUPPORTED, "padded path needs K > 0, M, N+15, K+15 < 2^30, batch <= 65535");
  const PaddedLayout L = padded_layout(q);
  const int64_t Kp = L.Kp, Np = L.Np, bA = L.bA, bB = L.bB;
  const bool copy_a = L.copy_a, copy_b = L.copy_b, copy_c = L.copy_c;
  const int64_t a_bytes = L.a_bytes, b_bytes = L.b_bytes, c_bytes = L.c_bytes;
  Problem g = q;
  hipStream_t s = (hipStream_t)scr.stream;
  if (a_bytes + b_bytes + c_bytes > 0) {
    void *w = nullptr;
    int rc = scr.take(kPadded, (size_t)(a_bytes + b_bytes + c_bytes), &w);
    if (rc) return rc;
    int8_t *Ap = (int8_t *)w, *Bp = Ap + a_bytes;
    int32_t *Cp = (int32_t *)(Bp + b_bytes);
    const PadArgs pa = {q.A, Ap, q.lda, bA > 1 ? q.sa : 0, q.M * Kp, q.M, q.K, q.M, Kp, bA};
    const PadArgs pb = {q.B, Bp, q.ldb, bB > 1 ? q.sb : 0, Kp * Np, q.K, q.N, Kp, Np, bB};
    // grid z = the operands copied; z = 0 takes the first of them
    const int64_t blocks_a = copy_a ? (q.M * (Kp / 16) + 255) / 256 : 0;
    const int64_t blocks_b = copy_b ? (Kp * (Np / 16) + 255) / 256 : 0;
    const int64_t blocks = blocks_a > blocks_b ? blocks_a : blocks_b;
    const int64_t ys = (copy_a && bA > bB) || !copy_b ? bA : bB;
    if (blocks > 0x7fffffff) return fail(VT_EUNSUPPORTED, "padded copy grid too large");
    if (blocks > 0) {
      hipLaunchKernelGGL(pad_i8_kernel, dim3((unsigned)blocks, (unsigned)ys, copy_a && copy_b ? 2 : 1),
                         dim3(256), 0, s, copy_a ? pa : pb, pb);
      VT_HIP_CHECK(hipGetLastError());
    }
    g = padded_inner(q, L, Ap, Bp, Cp);
  } else {
    g = padded_inner(q, L, nullptr, nullptr, nullptr);
  }
  int32_t v = 0, ks = 0;
  select_variant(g, true, &v, &ks);
  int rc = v == VT_VARIANT_GENERIC ? launch_generic(g, s) : launch_vector(g, v, ks, scr);
  if (rc || !copy_c) return rc;
  UnpadArgs u = {g.C, q.D, q.C, Np, q.ldd, q.ldc, q.M * Np, q.sd, q.sc, q.M, q.N};
  const int64_t cells = q.M * ((q.N + 3) / 4);   // one thread per 4 columns
  if ((cells + 255) / 256 > 0x7fffffff) return fail(VT_EUNSUPPORTED, "padded copy-out grid too large");
  dim3 ug((unsigned)((cells + 255) / 256), (unsigned)q.batch);
  if (q.D) hipLaunchKernelGGL(unpad_kernel<true>, ug, dim3(256), 0, s, u);
  else hipLaunchKernelGGL(unpad_kernel<false>, ug, dim3(256), 0, s, u);
  VT_HIP_CHECK(hipGetLastError());
  return VT_OK;
}

int launch_generic(const Problem &q, hipStream_t stream) {
  GenericArgs a;
  a.A = q.A; a.B = q.B; a.D = q.D; a.C = q.C;
  a.lda = q.lda; a.ldb = q.ldb; a.ldd = q.ldd; a.ldc = q.ldc;
  a.sa = q.sa; a.sb = q.sb; a.sd = q.sd; a.sc = q.sc;
  a.M = q.M; a.N = q.N; a.K = q.K; a.batch = q.batch;
  const int64_t gx = (q.N + 63) / 64;
  if (gx > 0x7fffffff) return fail(VT_EUNSUPPORTED, "N too large for the generic kernel");
  int64_t gy = (q.M + 3) / 4;
  if (gy > 65535) gy = 65535;
  int64_t gz = q.batch > 65535 ? 65535 : q.batch;
  hipLaunchKernelGGL(generic_kernel, dim3((unsigned)gx, (unsigned)gy, (unsigned)gz), dim3(256), 0,
                     stream, a);
  VT_HIP_CHECK(hipGetLastError());
  return VT_OK;
}


// The vector variants (operands already checked by vector_ok).
int launch_vector(const Problem &q, int32_t variant, int32_t k_split, Scratch &scr) {
  switch (variant) {
    case VT_VARIANT_MFMA_256x256: return launch_mfma<256, 256>(q, scr);
    case VT_VARIANT_MFMA_128x128: return launch_mfma128(q, scr);
    case VT_VARIANT_MFMA_256x128: return launch_mfma<256, 128>(q, scr);
    case VT_VARIANT_SKINNY: return launch_skinny(q, k_split, scr);
    default: return fail(VT_EINVAL, "variant %d is not a vector variant", (int)variant);
  }
}

// One validated vt_gemm_i8 problem and the kernel it runs.
struct GemmCall {
  Problem q;
  int32_t variant = VT_VARIANT_AUTO, k_split = 0;
  bool empty = false;   // nothing to compute (M, N or batch is 0)
};

// The host-side checks of vt_gemm_i8, in order, then the variant choice.
// Nothing here touches the device. With `pointers` false (vt_gemm_check) the
// operands are taken to be distinct allocations aligned to 16 bytes, as
// fresh device allocations are.
int prepare_gemm(const int8_t *A, const int8_t *B, const int32_t *D, int32_t *C, bool has_d,
                 bool pointers, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                 int64_t ldd, int64_t ldc, int64_t batch, int64_t stride_a, int64_t stride_b,
                 int64_t stride_d, int64_t stride_c, int32_t variant, int32_t k_split,
                 const char *who, GemmCall *out) {
  if (M < 0 || N < 0 || K < 0 || batch < 0)
    return fail(VT_EINVAL, "negative size (M=%lld N=%lld K=%lld batch=%lld)", (long long)M,
                (long long)N, (long long)K, (long long)batch);
  if (variant < 0 || variant >= VT_VARIANT_COUNT)
    return fail(VT_EINVAL, "unknown variant %d", (int)variant);
  if (k_split < 0 || k_split > 4096) return fail(VT_EINVAL, "k_split %d out of range", (int)k_split);
  if (stride_a < 0 || stride_b < 0 || stride_d < 0 || stride_c < 0)
    return fail(VT_EINVAL, "negative batch stride");
  if (M > (1ll << 40) || N > (1ll << 40) || K > (1ll << 40) || batch > (1ll << 31))
    return fail(VT_EINVAL, "size beyond 2^40 (batch beyond 2^31)");
  if (lda > (1ll << 40) || ldb > (1ll << 40) || ldd > (1ll << 40) || ldc > (1ll << 40) ||
      stride_a > (1ll << 56) || stride_b > (1ll << 56) || stride_d > (1ll << 56) ||
      stride_c > (1ll << 56))
    return fail(VT_EINVAL, "leading dimension beyond 2^40 or batch stride beyond 2^56");
  out->empty = M == 0 || N == 0 || batch == 0;
  if (out->empty) return VT_OK;
  if (pointers && !C) return fail(VT_EINVAL, "C is null");
  if (pointers && K > 0 && (!A || !B)) return fail(VT_EINVAL, "A or B is null");
  if (ldc < N) return fail(VT_EINVAL, "ldc=%lld < N=%lld", (long long)ldc, (long long)N);
  if (K > 0 && lda < K) return fail(VT_EINVAL, "lda=%lld < K=%lld", (long long)lda, (long long)K);
  if (K > 0 && ldb < N) return fail(VT_EINVAL, "ldb=%lld < N=%lld", (long long)ldb, (long long)N);
  if (has_d && ldd < N) return fail(VT_EINVAL, "ldd=%lld < N=%lld", (long long)ldd, (long long)N);
  if (batch > 1 && stride_c != 0 && (__int128)stride_c < (__int128)M * ldc)
    return fail(VT_EINVAL, "stride_c=%lld overlaps batches (M=%lld rows of ldc=%lld)",
                (long long)stride_c, (long long)M, (long long)ldc);
  if (batch > 1 && stride_c == 0) return fail(VT_EINVAL, "stride_c must be nonzero for batch > 1");
  if (pointers) {
    if (int rc = check_operand_overlap(A, B, D, C, M, N, K, lda, K, ldb, N, ldd, ldc, batch,
                                       stride_a, stride_b, stride_d, stride_c, who))
      return rc;
  }
  // Without pointers D stands for a distinct buffer: any non-null marker.
  const int32_t *d_mark = has_d ? (D ? D : (const int32_t *)(uintptr_t)16) : nullptr;
  Problem q = {A, B, d_mark, C, M, N, K, lda, ldb, ldd, ldc, batch,
               stride_a, stride_b, stride_d, stride_c};
  const bool vec = vector_ok(q);
  int32_t chosen = variant, ks = k_split;
  if (variant == VT_VARIANT_AUTO) {
    select_variant(q, vec, &chosen, &ks);
    if (k_split > 0) ks = k_split;
  } else if (variant != VT_VARIANT_GENERIC && variant != VT_VARIANT_PADDED) {
    if (!vec)
      return fail(VT_EUNSUPPORTED,
                  "variant %s needs N%%16==0, K%%16==0 (K>0), lda/ldb/strides multiples of 16 "
                  "and 16-byte aligned A, B",
                  kVariants[variant].name);
    if (variant == VT_VARIANT_SKINNY && M > kSkinnyMaxM)
      return fail(VT_EUNSUPPORTED, "variant skinny needs M <= %d (M=%lld)", kSkinnyMaxM,
                  (long long)M);
    if (variant != VT_VARIANT_SKINNY && !mfma_addressable(q))
      return fail(VT_EUNSUPPORTED,
                  "variant %s needs 256*lda and 64*ldb below 2^32 (lda=%lld ldb=%lld)",
                  kVariants[variant].name, (long long)lda, (long long)ldb);
  }
  if (chosen != VT_VARIANT_GENERIC && chosen != VT_VARIANT_PADDED && !vec)
    return fail(VT_EUNSUPPORTED, "internal: vector variant selected for an unaligned problem");
  if (chosen == VT_VARIANT_PADDED && K == 0) chosen = VT_VARIANT_GENERIC;   // C = D (or 0)
  if (chosen == VT_VARIANT_PADDED && !padded_fits(q))
    return fail(VT_EUNSUPPORTED, "padded path needs K > 0, M, N+15, K+15 < 2^30, batch <= 65535");
  out->q = q;
  out->variant = chosen;
  out->k_split = ks;
  return VT_OK;
}

int launch_gemm(const GemmCall &c, Scratch &scr) {
  if (c.variant == VT_VARIANT_GENERIC) return launch_generic(c.q, (hipStream_t)scr.stream);
  if (c.variant == VT_VARIANT_PADDED) return launch_padded(c.q, scr);
  return launch_vector(c.q, c.variant, c.k_split, scr);
}

// Dynamic LDS beyond the default for the kernels that need it.
void set_kernel_attributes(DeviceState &st) {
  const std::pair<const void *, int> need[] = {
      {(const void *)skinny_kernel<kSkinnyNB, kSkinnyWaves, kSkinnyU, 1, true>, kMaxSkinnyLds},
      {(const void *)skinny_kernel<kSkinnyNB, kSkinnyWaves, kSkinnyU, 1, false>, kMaxSkinnyLds},
      {(const void *)skinny_kernel<kSkinnyNB, kSkinnyWaves, kSkinnyU, 2, true>, kMaxSkinnyLds},
      {(const void *)skinny_kernel<kSkinnyNB, kSkinnyWaves, kSkinnyU, 2, false>, kMaxSkinnyLds},
      {(const void *)skinny_kernel<kSkinnyNB, kSkinnyWaves, kSkinnyU, 4, true>, kMaxSkinnyLds},
      {(const void *)skinny_kernel<kSkinnyNB, kSkinnyWaves, kSkinnyU, 4, false>, kMaxSkinnyLds},
      {(const void *)skinny_kernel<kSkinnyNB, kSkinnyWaves, kSkinnyU, 1, true, true>, kMaxSkinnyLds},
      {(const void *)skinny_kernel<kSkinnyNB, kSkinnyWaves, kSkinnyU, 1, false, true>, kMaxSkinnyLds},
      {(const void *)replay_kernel, kMaxReplayLds + 256},
  };
  for (const auto &n : need) {
    const hipError_t e =
        hipFuncSetAttribute(n.first, hipFuncAttributeMaxDynamicSharedMemorySize, n.second);
    if (e != hipSuccess && st.attr_err == hipSuccess) st.attr_err = e;
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------

extern "C" {

int vt_abi_version(void) { return VT_ABI_VERSION; }

int vt_replay_i8(const int32_t *program, int64_t n_ops, const int8_t *A, const int8_t *B,
                 int32_t *C, int64_t m, int64_t n, int64_t k, int64_t scratchpad_rows,
                 int64_t accumulator_rows, int32_t *status, void *stream) {
  g_err.clear();
  if (m <= 0 || n <= 0 || k <= 0 || n_ops < 0)
    return fail(VT_EINVAL, "replay sizes must be positive (m=%lld n=%lld k=%lld ops=%lld)",
                (long long)m, (long long)n, (long long)k, (long long)n_ops);
  if (m * k > INT32_MAX || k * n > INT32_MAX || m * n > INT32_MAX || n_ops > (1 << 28))
    return fail(VT_EINVAL, "replay extents beyond the int32 indexing range");
  if (scratchpad_rows < 16 || accumulator_rows < 16)
    return fail(VT_EINVAL, "scratchpad and accumulator need at least 16 rows");
  if (scratchpad_rows * 16 + accumulator_rows * 64 > kMaxReplayLds)
    return fail(VT_EUNSUPPORTED,
                "scratchpad (%lld rows) and accumulator (%lld rows) exceed the %d-byte LDS budget",
                (long long)scratchpad_rows, (long long)accumulator_rows, kMaxReplayLds);
  if (!A || !B || !C || !status || (n_ops > 0 && !program))
    return fail(VT_EINVAL, "replay pointer is null");
  int dev = 0;
  DeviceState *st = nullptr;
  int rc = current_device(&dev, &st);
  if (rc) return rc;
  ReplayArgs a;
  a.prog = program;
  a.n_ops = (int)n_ops;
  a.A = A;
  a.B = B;
  a.C = C;
  a.size_a = m * k;
  a.size_b = k * n;
  a.size_c = m * n;
  a.spad_rows = (int)scratchpad_rows;
  a.acc_rows = (int)accumulator_rows;
  a.status = status;
  const size_t lds = (size_t)(scratchpad_rows * 16 + accumulator_rows * 64 + 256);
  hipLaunchKernelGGL(replay_kernel, dim3(1), dim3(256), lds, (hipStream_t)stream, a);
  VT_HIP_CHECK(hipGetLastError());
  return VT_OK;
}

const char *vt_last_error(void) { return g_err.c_str(); }

const char *vt_variant_name(int32_t variant) {
  if (variant < 0 || variant >= VT_VARIANT_COUNT) return nullptr;
  return kVariants[variant].name;
}

int vt_variant_info(int32_t variant, int32_t *tile_m, int32_t *tile_n, int32_t *tile_k,
                    int32_t *threads, int32_t *lds_bytes) {
  if (variant <= 0 || variant >= VT_VARIANT_COUNT)
    return fail(VT_EINVAL, "unknown variant %d", (int)variant);
  const VariantInfo &v = kVariants[variant];
  if (tile_m) *tile_m = v.tile_m;
  if (tile_n) *tile_n = v.tile_n;
  if (tile_k) *tile_k = v.tile_k;
  if (threads) *threads = v.threads;
  if (lds_bytes) *lds_bytes = v.lds_bytes;
  return VT_OK;
}

int vt_gemm_select(int64_t M, int64_t N, int64_t K, int64_t batch, int64_t lda, int64_t ldb,
                   int32_t flags, int32_t *variant_out, int32_t *k_split_out) {
  if (!variant_out || !k_split_out) return fail(VT_EINVAL, "null output pointer");
  if (M < 0 || N < 0 || K < 0 || batch < 0) return fail(VT_EINVAL, "negative size");
  if (flags & ~(VT_SELECT_ALIGNED | VT_SELECT_B_SHARED))
    return fail(VT_EINVAL, "unknown vt_gemm_select flags 0x%x", (unsigned)flags);
  Problem q = {};
  q.M = M; q.N = N; q.K = K; q.batch = batch; q.lda = lda; q.ldb = ldb;
  q.sa = M * lda; q.sc = M * N; q.ldc = N;
  q.sb = (flags & VT_SELECT_B_SHARED) || batch <= 1 ? 0 : K * ldb;
  const bool vec = (flags & VT_SELECT_ALIGNED) && q.N % 16 == 0 && q.K % 16 == 0 && q.K > 0 &&
                   lda % 16 == 0 && ldb % 16 == 0;
  return select_variant(q, vec, variant_out, k_split_out);
}

int vt_device_count(void) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess) return 0;
  int n = 0;
  for (int d = 0; d < count; ++d) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, d) == hipSuccess &&
        strncmp(prop.gcnArchName, "gfx950", 6) == 0)
      ++n;
  }
  return n;
}

static_assert(sizeof(vt_device_info) == 624, "vt_device_info layout is part of the ABI");

int vt_device_query(int32_t device, vt_device_info *info, int64_t info_size) {
  if (info == nullptr) return fail(VT_EINVAL, "vt_device_query: info is NULL");
  if (info_size != (int64_t)sizeof(vt_device_info))
    return fail(VT_EINVAL, "vt_device_query: info_size %lld != sizeof(vt_device_info) %zu",
                (long long)info_size, sizeof(vt_device_info));
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0)
    return fail(VT_ENODEV, "no HIP device available");
  int dev = device;
  if (dev < 0) VT_HIP_CHECK(hipGetDevice(&dev));
  if (dev >= count)
    return fail(VT_EINVAL, "vt_device_query: device %d of %d", dev, count);
  hipDeviceProp_t prop;
  VT_HIP_CHECK(hipGetDeviceProperties(&prop, dev));
  memset(info, 0, sizeof *info);
  snprintf(info->name, sizeof info->name, "%s", prop.name);
  snprintf(info->arch, sizeof info->arch, "%s", prop.gcnArchName);
  snprintf(info->code_object_arch, sizeof info->code_object_arch, "%s", "gfx950");
  info->total_memory_bytes = (int64_t)prop.totalGlobalMem;
  info->l2_cache_bytes = prop.l2CacheSize;
  info->lds_per_workgroup_bytes = (int64_t)(prop.sharedMemPerBlockOptin > prop.sharedMemPerBlock
                                                ? prop.sharedMemPerBlockOptin
                                                : prop.sharedMemPerBlock);
  info->lds_per_cu_bytes = (int64_t)prop.maxSharedMemoryPerMultiProcessor;
  info->compute_units = prop.multiProcessorCount;
  info->wavefront_size = prop.warpSize;
  info->max_threads_per_workgroup = prop.maxThreadsPerBlock;
  info->max_clock_khz = prop.clockRate;
  info->memory_clock_khz = prop.memoryClockRate;
  info->memory_bus_width_bits = prop.memoryBusWidth;
  info->pci_domain = prop.pciDomainID;
  info->pci_bus = prop.pciBusID;
  info->pci_device = prop.pciDeviceID;
  VT_HIP_CHECK(hipRuntimeGetVersion(&info->hip_runtime_version));
  VT_HIP_CHECK(hipDriverGetVersion(&info->hip_driver_version));
  // gcnArchName carries target features after the ISA name ("gfx950:sramecc+:xnack-").
  const size_t isa = strcspn(prop.gcnArchName, ":");
  info->supported = isa == 6 && strncmp(prop.gcnArchName, "gfx950", 6) == 0;
  return VT_OK;
}

int vt_sync(void *stream) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0)
    return fail(VT_ENODEV, "no HIP device available");
  VT_HIP_CHECK(hipStreamSynchronize((hipStream_t)stream));
  VT_HIP_CHECK(hipGetLastError());
  return VT_OK;
}

int vt_gemm_i8(const int8_t *A, const int8_t *B, const int32_t *D, int32_t *C, int64_t M,
               int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldd, int64_t ldc,
               int64_t batch, int64_t stride_a, int64_t stride_b, int64_t stride_d,
               int64_t stride_c, int32_t variant, int32_t k_split, void *stream) {
  g_err.clear();
  GemmCall c;
  int rc = prepare_gemm(A, B, D, C, D != nullptr, true, M, N, K, lda, ldb, ldd, ldc, batch,
                        stride_a, stride_b, stride_d, stride_c, variant, k_split, "vt_gemm_i8",
                        &c);
  if (rc || c.empty) return rc;
  int dev = 0;
  DeviceState *st = nullptr;
  rc = current_device(&dev, &st);
  if (rc) return rc;
  Scratch scr;
  scr.st = st;
  scr.stream = stream;
  return launch_gemm(c, scr);
}

int vt_gemm_i8_noalloc(const int8_t *A, const int8_t *B, const int32_t *D, int32_t *C,
                       int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldd,
                       int64_t ldc, int64_t batch, int64_t stride_a, int64_t stride_b,
                       int64_t stride_d, int64_t stride_c, int32_t variant, int32_t k_split,
                       void *stream) {
  g_err.clear();
  GemmCall c;
  int rc = prepare_gemm(A, B, D, C, D != nullptr, true, M, N, K, lda, ldb, ldd, ldc, batch,
                        stride_a, stride_b, stride_d, stride_c, variant, k_split,
                        "vt_gemm_i8_noalloc", &c);
  if (rc || c.empty) return rc;
  // Refused before anything is launched when the scratch array is too small.
  const int64_t need = scratch_need(c.q, c.variant, c.k_split);
  if (need > (int64_t)kScratchBytes)
    return fail(VT_EUNSUPPORTED,
                "vt_gemm_i8_noalloc: this call needs %lld bytes of scratch; the static scratch "
                "array holds %zu (use vt_gemm_i8)",
                (long long)need, kScratchBytes);
  int dev = 0;
  DeviceState *st = nullptr;
  rc = current_device(&dev, &st);
  if (rc) return rc;
  // This device's address of the array, looked up when the device was
  // first used (each device has its own copy).
  if (!st->scratch)
    return fail(VT_EHIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                hipGetErrorString(st->scratch_err));
  Scratch scr;
  scr.st = st;
  scr.stream = stream;
  scr.fixed = st->scratch;
  return launch_gemm(c, scr);
}

int vt_gemm_check(int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldd,
                  int64_t ldc, int64_t batch, int64_t stride_a, int64_t stride_b, int64_t stride_d,
                  int64_t stride_c, int32_t has_d, int32_t variant, int32_t k_split,
                  int32_t *variant_out, int32_t *k_split_out, int64_t *scratch_bytes_out) {
  g_err.clear();
  GemmCall c;
  int rc = prepare_gemm(nullptr, nullptr, nullptr, nullptr, has_d != 0, false, M, N, K, lda, ldb,
                        ldd, ldc, batch, stride_a, stride_b, stride_d, stride_c, variant, k_split,
                        "vt_gemm_check", &c);
  if (rc) return rc;
  if (variant_out) *variant_out = c.empty ? VT_VARIANT_AUTO : c.variant;
  // The K split that launches: the skinny kernel's slice count, or the MFMA
  // kernels' (1 reported as 0: no split); padded chooses its own for the
  // padded shape.
  int32_t ks = 0;
  if (!c.empty && c.variant == VT_VARIANT_SKINNY)
    ks = skinny_geometry<kSkinnyNB, kSkinnyWaves, kSkinnyU>(c.q, c.k_split).ks;
  else if (!c.empty) {
    const int mks = mfma_split_for(c.q, c.variant);
    ks = mks > 1 ? mks : 0;
  }
  if (k_split_out) *k_split_out = ks;
  if (scratch_bytes_out) *scratch_bytes_out = c.empty ? 0 : scratch_need(c.q, c.variant, c.k_split);
  return VT_OK;
}

int64_t vt_packed_b_size(int64_t K, int64_t N) {
  if (K < 0 || N < 0 || N % 16 != 0 || K >= (1ll << 30) || N >= (1ll << 30))
    return fail(VT_EINVAL, "packed B needs 0 <= K < 2^30 and 0 <= N < 2^30 with N %% 16 == 0 "
                "(K=%lld N=%lld)", (long long)K, (long long)N);
  return N * packed_kbt(K) * 64;
}

int vt_pack_b_i8(const int8_t *B, int8_t *Bp, int64_t K, int64_t N, int64_t ldb, int64_t batch,
                 int64_t stride_b, int64_t stride_bp, void *stream) {
  g_err.clear();
  if (K < 0 || N < 0 || batch < 0) return fail(VT_EINVAL, "negative size");
  const int64_t size = vt_packed_b_size(K, N);
  if (size < 0) return (int)size;
  if (K == 0 || N == 0 || batch == 0) return VT_OK;
  if (!B || !Bp) return fail(VT_EINVAL, "B or Bp is null");
  if (ldb < N) return fail(VT_EINVAL, "ldb=%lld < N=%lld", (long long)ldb, (long long)N);
  if (ldb % 16 || stride_b % 16 || stride_bp % 16 || !aligned16(B) || !aligned16(Bp))
    return fail(VT_EUNSUPPORTED, "pack needs ldb and strides multiples of 16 and 16-byte aligned B, Bp");
  if (stride_b < 0 || stride_bp < 0) return fail(VT_EINVAL, "negative batch stride");
  if (batch > 1 && stride_bp < size)
    return fail(VT_EINVAL, "stride_bp=%lld overlaps packed batches (size %lld)",
                (long long)stride_bp, (long long)size);
  if (batch > 65535 || (N + 255) / 256 > 65535)
    return fail(VT_EUNSUPPORTED, "pack grid too large (batch=%lld N=%lld)", (long long)batch,
                (long long)N);
  if (ldb > (1ll << 40) || stride_b > (1ll << 56) || stride_bp > (1ll << 56))
    return fail(VT_EINVAL, "ldb beyond 2^40 or batch stride beyond 2^56");
  if ((__int128)(K - 1) * ldb + N >= ((__int128)1 << 40))
    return fail(VT_EINVAL, "B extent beyond 2^40");
  {
    Extent eb, ep;
    if (!operand_extent(B, batch, stride_b, K, ldb, N, 1, &eb) ||
        !operand_extent(Bp, batch, stride_bp, 1, 0, size, 1, &ep))
      return fail(VT_EINVAL, "vt_pack_b_i8: extent beyond 2^56 bytes");
    if (overlaps(eb, ep)) return fail(VT_EINVAL, "vt_pack_b_i8: Bp overlaps B in memory");
  }
  int dev = 0;
  DeviceState *st = nullptr;
  int rc = current_device(&dev, &st);
  if (rc) return rc;
  PackArgs a;
  a.B = B; a.Bp = Bp; a.ldb = ldb; a.sb = stride_b; a.sbp = stride_bp;
  a.K = (int)K; a.N = (int)N; a.kbt = (int)packed_kbt(K);
  hipLaunchKernelGGL(pack_b_kernel, dim3((unsigned)a.kbt, (unsigned)((N + 255) / 256), (unsigned)batch),
                     dim3(256), 0, (hipStream_t)stream, a);
  VT_HIP_CHECK(hipGetLastError());
  return VT_OK;
}

int vt_gemm_i8_packed(const int8_t *A, const int8_t *Bp, const int32_t *D, int32_t *C, int64_t M,
                      int64_t N, int64_t K, int64_t lda, int64_t ldd, int64_t ldc, int64_t batch,
                      int64_t stride_a, int64_t stride_bp, int64_t stride_d, int64_t stride_c,
                      int32_t k_split, void *stream) {
  g_err.clear();
  if (M < 0 || N < 0 || K < 0 || batch < 0)
    return fail(VT_EINVAL, "negative size (M=%lld N=%lld K=%lld batch=%lld)", (long long)M,
                (long long)N, (long long)K, (long long)batch);
  if (k_split < 0 || k_split > 4096) return fail(VT_EINVAL, "k_split %d out of range", (int)k_split);
  if (stride_a < 0 || stride_bp < 0 || stride_d < 0 || stride_c < 0)
    return fail(VT_EINVAL, "negative batch stride");
  if (lda > (1ll << 40) || ldd > (1ll << 40) || ldc > (1ll << 40) || batch > (1ll << 31) ||
      stride_a > (1ll << 56) || stride_bp > (1ll << 56) || stride_d > (1ll << 56) ||
      stride_c > (1ll << 56))
    return fail(VT_EINVAL, "leading dimension beyond 2^40, batch beyond 2^31 or stride beyond 2^56");
  if (M == 0 || N == 0 || batch == 0) return VT_OK;
  if (!C) return fail(VT_EINVAL, "C is null");
  if (K > 0 && (!A || !Bp)) return fail(VT_EINVAL, "A or Bp is null");
  if (ldc < N) return fail(VT_EINVAL, "ldc=%lld < N=%lld", (long long)ldc, (long long)N);
  if (K > 0 && lda < K) return fail(VT_EINVAL, "lda=%lld < K=%lld", (long long)lda, (long long)K);
  if (D && ldd < N) return fail(VT_EINVAL, "ldd=%lld < N=%lld", (long long)ldd, (long long)N);
  if (batch > 1 && (__int128)stride_c < (__int128)M * ldc)
    return fail(VT_EINVAL, "stride_c=%lld overlaps batches (M=%lld rows of ldc=%lld)",
                (long long)stride_c, (long long)M, (long long)ldc);
  if (M >= (1ll << 30) || N >= (1ll << 30) || K >= (1ll << 30))
    return fail(VT_EINVAL, "size beyond 2^30");
  // packed B: one contiguous block of packed_b_size bytes per batch
  if (int rc = check_operand_overlap(A, Bp, D, C, M, N, K, lda, 1, 0,
                                     N * ((K + 63) / 64) * 64, ldd, ldc, batch, stride_a,
                                     stride_bp, stride_d, stride_c, "vt_gemm_i8_packed"))
    return rc;
  if (N % 16 || K % 16)
    return fail(VT_EUNSUPPORTED, "packed B needs N %% 16 == 0 and K %% 16 == 0 (N=%lld K=%lld)",
                (long long)N, (long long)K);
  if (K > 0 && (lda % 16 || stride_a % 16 || stride_bp % 16 || !aligned16(A) || !aligned16(Bp)))
    return fail(VT_EUNSUPPORTED,
                "packed GEMM needs lda and strides multiples of 16 and 16-byte aligned A, Bp");
  if (batch > 65535) return fail(VT_EUNSUPPORTED, "packed GEMM supports batch <= 65535");
  int dev = 0;
  DeviceState *st = nullptr;
  int rc = current_device(&dev, &st);
  if (rc) return rc;
  Problem q = {A, Bp, D, C, M, N, K, lda, 0, ldd, ldc, batch, stride_a, stride_bp, stride_d, stride_c};
  Scratch scr;
  scr.st = st;
  scr.stream = stream;
  if (K == 0) return launch_generic(q, (hipStream_t)stream);   // C = D (or 0)
  // Rows on the persistent DMA kernel when there are enough whole 256-row
  // tiles (all rows, unless the partial last tile row would add a round), or
  // all rows on its 256x128 form (packed_dma128_fits);
  // more than 64 remaining rows on 128x128 tiles; up to 64 rows, or tiles
  // whose offsets do not fit 32 bits, in groups of up to 64 rows on the
  // decode kernel, each group streaming B once.
  if (packed_dma_rows(q) == 0 && packed_dma128_fits(q))
    return launch_packed_dma128(q, (hipStream_t)stream, st->num_cus);
  int64_t r_first = 0;
  if (const int64_t rows = packed_dma_rows(q)) {
    rc = launch_packed_dma(q, rows, (hipStream_t)stream, st->num_cus);
    if (rc) return rc;
    r_first = rows;
  }
  if (M - r_first > kSkinnyMaxM && packed_tiles_fit(q)) {
    Problem g = q;
    g.A = A + r_first * lda;
    g.C = C + r_first * ldc;
    g.D = D ? D + r_first * ldd : nullptr;
    g.M = M - r_first;
    g.ldb = packed_kbt(K);
    return launch_mfma<128, 128, true>(g, scr);
  }
  for (int64_t r0 = r_first; r0 < M; r0 += kSkinnyMaxM) {
    Problem g = q;
    g.A = A + r0 * lda;
    g.C = C + r0 * ldc;
    g.D = D ? D + r0 * ldd : nullptr;
    g.M = M - r0 < kSkinnyMaxM ? M - r0 : kSkinnyMaxM;
    rc = launch_packed_rows(g, k_split, scr);
    if (rc) return rc;
  }
  return VT_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Run-time compiled loop-nest kernels (hipRTC)
// ---------------------------------------------------------------------------

// A gfx950 code object compiled from source, and its module / function on
// every device it has been launched on.
struct vt_rtc_program {
  std::string kernel;
  std::vector<char> code;
  std::mutex mu;
  std::map<int, std::pair<hipModule_t, hipFunction_t>> loaded;
};

extern "C" {

int vt_rtc_compile(const char *source, const char *kernel_name, vt_rtc_program **out) {
  g_err.clear();
  if (!source || !kernel_name || !out) return fail(VT_EINVAL, "vt_rtc_compile: null argument");
  *out = nullptr;
  if (!kernel_name[0] || strlen(kernel_name) > 255)
    return fail(VT_EINVAL, "vt_rtc_compile: bad kernel name");
  hiprtcProgram prog;
  hiprtcResult r = hiprtcCreateProgram(&prog, source, "loopnest.hip", 0, nullptr, nullptr);
  if (r != HIPRTC_SUCCESS) return fail(VT_EHIP, "hiprtcCreateProgram: %s", hiprtcGetErrorString(r));
  // Same code-generation rules as the library's own kernels: gfx950, no
  // packed FP32 instructions; no FMA contraction, so floating-point loop
  // nests round like the C they are emitted from; signed overflow wraps
  // (two's complement) instead of being undefined, so an integer nest's
  // stores keep the low bits of the exact result.
  const char *opts[] = {"--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
                        "-fwrapv", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
  r = hiprtcCompileProgram(prog, (int)(sizeof opts / sizeof opts[0]), opts);
  if (r != HIPRTC_SUCCESS) {
    size_t n = 0;
    std::string log;
    if (hiprtcGetProgramLogSize(prog, &n) == HIPRTC_SUCCESS && n > 0) {
      log.resize(n);
      hiprtcGetProgramLog(prog, &log[0]);
    }
    hiprtcDestroyProgram(&prog);
    if (log.size() > 400) log = log.substr(0, 400) + "...";
    return fail(VT_EINVAL, "hiprtcCompileProgram: %s: %s", hiprtcGetErrorString(r), log.c_str());
  }
  size_t size = 0;
  r = hiprtcGetCodeSize(prog, &size);
  std::vector<char> code(size);
  if (r == HIPRTC_SUCCESS && size > 0) r = hiprtcGetCode(prog, code.data());
  hiprtcDestroyProgram(&prog);
  if (r != HIPRTC_SUCCESS || size == 0)
    return fail(VT_EHIP, "hiprtcGetCode: %s", hiprtcGetErrorString(r));
  vt_rtc_program *p = new vt_rtc_program;
  p->kernel = kernel_name;
  p->code = std::move(code);
  *out = p;
  return VT_OK;
}

int64_t vt_rtc_code_size(const vt_rtc_program *p) {
  if (!p) return fail(VT_EINVAL, "vt_rtc_code_size: null program");
  return (int64_t)p->code.size();
}

int vt_rtc_launch(vt_rtc_program *p, uint32_t grid_x, uint32_t grid_y, uint32_t grid_z,
                  uint32_t block_x, uint32_t block_y, uint32_t block_z, void **args,
                  void *stream) {
  g_err.clear();
  if (!p) return fail(VT_EINVAL, "vt_rtc_launch: null program");
  if (!grid_x || !grid_y || !grid_z || !block_x || !block_y || !block_z ||
      (uint64_t)block_x * block_y * block_z > 1024 || grid_y > 65535 || grid_z > 65535)
    return fail(VT_EINVAL, "vt_rtc_launch: bad launch shape");
  int dev = 0;
  DeviceState *st = nullptr;
  int rc = current_device(&dev, &st);
  if (rc) return rc;
  hipFunction_t fn = nullptr;
  {
    std::lock_guard<std::mutex> lk(p->mu);
    auto it = p->loaded.find(dev);
    if (it == p->loaded.end()) {
      hipModule_t mod = nullptr;
      VT_HIP_CHECK(hipModuleLoadData(&mod, p->code.data()));
      hipError_t e = hipModuleGetFunction(&fn, mod, p->kernel.c_str());
      if (e != hipSuccess) {
        (void)hipModuleUnload(mod);
        return fail(VT_EINVAL, "kernel %s not in the compiled module: %s", p->kernel.c_str(),
                    hipGetErrorString(e));
      }
      p->loaded[dev] = std::make_pair(mod, fn);
    } else {
      fn = it->second.second;
    }
  }
  VT_HIP_CHECK(hipModuleLaunchKernel(fn, grid_x, grid_y, grid_z, block_x, block_y, block_z, 0,
                                     (hipStream_t)stream, args, nullptr));
  return VT_OK;
}

void vt_rtc_release(vt_rtc_program *p) {
  if (!p) return;
  int cur = -1;
  const bool have_cur = hipGetDevice(&cur) == hipSuccess;
  for (auto &kv : p->loaded) {
    if (hipSetDevice(kv.first) == hipSuccess) (void)hipModuleUnload(kv.second.first);
  }
  if (have_cur && !p->loaded.empty()) (void)hipSetDevice(cur);
  delete p;
}

}  // extern "C"
