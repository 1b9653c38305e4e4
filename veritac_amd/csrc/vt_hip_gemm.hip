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
//   gemm_mfma_kernel<BM,BN>  compute-bound tiles. 256 threads = 4 waves in a
//       2x2 grid, each wave owns a (BM/2)x(BN/2) block of 32x32 accumulators
//       fed by v_mfma_i32_32x32x32_i8. A/B k-slices of 64 bytes are staged
//       global -> VGPR -> LDS (double buffer, one LDS-only barrier per step,
//       next slice's global loads in flight during the MFMAs). A is stored
//       [m][k] and read with ds_read_b128; B stays row-major [k][n] in LDS and
//       is read into the MFMA operand layout with ds_read_b64_tr_b8 (gfx950's
//       transposing LDS read), so B is never transposed in memory. 16-byte
//       chunks are XOR-swizzled so the LDS reads are bank-conflict free.
//       Workgroup ids are remapped so consecutive tiles share an XCD (and its
//       L2), then grouped along M.
//   skinny_kernel<NB>  M <= 16 (decode). Bandwidth-bound: each workgroup
//       streams an NB-column slab of B exactly once over a K slice, U slices
//       of 64 rows in flight in registers, LDS double buffer, the A slice
//       resident in LDS, v_mfma_i32_16x16x64_i8 with M padded to 16 by zero
//       rows. K slices are reduced by the last-arriving workgroup of each
//       column slab (int32 partials in a workspace, device-scope counter).
//   generic_kernel  any shape, stride or alignment; one thread per output,
//       int32 VALU. Used where the vector kernels' alignment rules fail.
//
// Tails: rows of A past M and columns of B past N are read from clamped (valid)
// addresses and their outputs are never stored; k past K reads A as zero, so
// the clamped B rows there contribute nothing.

#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <map>
#include <mutex>
#include <string>
#include <utility>

#include "vt_hip_gemm.h"

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

// Swizzle of the 16-byte chunk index of a row-major [k][n] B slice with
// `chunks` 16-byte chunks per row: keeps the 8 rows one ds_read_b64_tr_b8
// touches in 8 distinct 16-byte bank groups.
template <int CHUNKS>
__device__ __forceinline__ int b_swz(int row) {
  static_assert(CHUNKS >= 4, "B slice needs at least 4 chunks per row");
  return CHUNKS >= 8 ? (row & 7) : ((row >> 1) & 3);
}

// A slice [m][64 bytes]: chunk c of row r lives at c ^ ((r >> 1) & 3).
__device__ __forceinline__ int a_off(int row, int c) {
  return row * 64 + ((c ^ ((row >> 1) & 3)) << 4);
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
};

template <int BM, int BN, bool EDGE, bool HAS_D>
__global__ __launch_bounds__(256, 1) void gemm_mfma_kernel(GemmArgs p) {
  constexpr int BK = 64;
  constexpr int WTM = BM / 2, WTN = BN / 2;   // wave tile (2x2 waves)
  constexpr int MI = WTM / 32, NI = WTN / 32; // 32x32 blocks per wave
  constexpr int BCH = BN / 16;                // 16-byte chunks per B row
  constexpr int CA = BM * (BK / 16) / 256;    // A chunks per thread per slice
  constexpr int CB = BK * BCH / 256;          // B chunks per thread per slice
  constexpr int A_BYTES = BM * BK, B_BYTES = BK * BN;
  static_assert(CA >= 1 && CB >= 1 && BCH >= 8, "tile too small");

  __shared__ __attribute__((aligned(16))) int8_t smem[2 * (A_BYTES + B_BYTES)];
  int8_t *const As0 = smem;                  // A slice buffer b at As0 + b*A_BYTES
  int8_t *const Bs0 = smem + 2 * A_BYTES;    // B slice buffer b at Bs0 + b*B_BYTES

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
  const int8_t *Ab = p.A + bidx * p.sa;
  const int8_t *Bb = p.B + bidx * p.sb;

  // Per-thread global source addresses for one 64-deep k slice.
  const int8_t *a_src[CA];
  int a_lds[CA], a_k[CA];
#pragma unroll
  for (int i = 0; i < CA; ++i) {
    const int row = (tid >> 2) + 64 * i, c = tid & 3;
    int grow = m0 + row;
    if (EDGE) grow = min(grow, M - 1);
    a_src[i] = Ab + (int64_t)grow * p.lda + c * 16;
    a_lds[i] = a_off(row, c);
    a_k[i] = c * 16;
  }
  int b_row[CB], b_col[CB], b_lds[CB];
#pragma unroll
  for (int i = 0; i < CB; ++i) {
    const int row = tid / BCH + (256 / BCH) * i, c = tid % BCH;
    int col = n0 + c * 16;
    if (EDGE) col = min(col, N - 16);
    b_row[i] = row;
    b_col[i] = col;
    b_lds[i] = row * BN + ((c ^ b_swz<BCH>(row)) << 4);
  }

  v4i ra[CA], rb[CB];
  auto load_slice = [&](int kt) {
    const int k0 = kt * BK;
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      if (EDGE && k0 + a_k[i] >= K) {
        ra[i] = v4i{0, 0, 0, 0};
      } else {
        ra[i] = *(const v4i *)(a_src[i] + k0);
      }
    }
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      int krow = k0 + b_row[i];
      if (EDGE) krow = min(krow, K - 1);
      rb[i] = *(const v4i *)(Bb + (int64_t)krow * p.ldb + b_col[i]);
    }
  };
  auto store_slice = [&](int buf) {
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
      const int nc = (wn * WTN + ni * 32) / 16 + (g & 1);
      const int r0 = ks * 32 + (g >> 1) * 16 + (j >> 1);
      b_frag[ks][ni] = r0 * BN + ((nc ^ b_swz<BCH>(r0)) << 4) + (j & 1) * 8;
    }

  const int KT = (K + BK - 1) / BK;
  load_slice(0);
  store_slice(0);
  lds_barrier();
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    const int8_t *As = As0 + cur * A_BYTES;
    const int8_t *Bs = Bs0 + cur * B_BYTES;
    if (kt + 1 < KT) load_slice(kt + 1);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      v4i a[MI], b[NI];
#pragma unroll
      for (int mi = 0; mi < MI; ++mi) a[mi] = ld_lds_b128(As, a_frag[ks][mi]);
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) {
        const v2i lo = ld_lds_tr8(Bs, b_frag[ks][ni]);
        const v2i hi = ld_lds_tr8(Bs, b_frag[ks][ni] + 8 * BN);
        b[ni] = v4i{lo.x, lo.y, hi.x, hi.y};
      }
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni)
          acc[mi][ni] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[mi], b[ni], acc[mi][ni], 0, 0, 0);
    }
    if (kt + 1 < KT) store_slice(cur ^ 1);
    lds_barrier();
  }

  // Epilogue. 32x32 accumulator layout: element e of lane l is
  // row 8*(e/4) + 4*(l/32) + e%4, column l%32.
  int32_t *Cb = p.C + bidx * p.sc;
  const int32_t *Db = HAS_D ? p.D + bidx * p.sd : nullptr;
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) {
      const int col = n0 + wn * WTN + ni * 32 + (lane & 31);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = m0 + wm * WTM + mi * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
        if (!EDGE || (row < M && col < N)) {
          int32_t v = acc[mi][ni][e];
          if (HAS_D) v = add_wrap(v, Db[(int64_t)row * p.ldd + col]);
          Cb[(int64_t)row * p.ldc + col] = v;
        }
      }
    }
}

// ---------------------------------------------------------------------------
// Skinny (decode) kernel: M <= 16
// ---------------------------------------------------------------------------

struct SkinnyArgs {
  const int8_t *A;
  const int8_t *B;
  const int32_t *D;
  int32_t *C;
  int64_t lda, ldb, ldd, ldc;
  int64_t sa, sb, sd, sc;
  int M, N, K;
  int tiles_n;     // ceil(N / NB)
  int k_split;     // K slices per column slab
  int k_chunk;     // rows per slice (multiple of 64)
  int32_t *ws;     // [batch][k_split][16][N] partials (k_split > 1)
  int *counters;   // [batch][tiles_n] arrival counters, zero between launches
};

constexpr int SKINNY_U = 8;   // 64-row B slices in flight per thread

template <int NB, bool HAS_D>
__global__ __launch_bounds__(256) void skinny_kernel(SkinnyArgs p) {
  constexpr int BCH = NB / 16;          // 16-byte chunks per B row (= n-blocks)
  constexpr int CB = 64 * BCH / 256;    // B chunks per thread per slice
  constexpr int NBW = BCH / 4;          // n-blocks per wave
  constexpr int U = SKINNY_U;
  static_assert(CB >= 1 && NBW >= 1, "NB must be >= 64");

  extern __shared__ __attribute__((aligned(16))) int8_t dsmem[];
  const int a_stride = p.k_chunk + 16;  // +16 bytes: rows land in distinct banks
  int8_t *As = dsmem;
  int8_t *const Bs0 = dsmem + 16 * a_stride;   // B slice buffer b at Bs0 + b*64*NB

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tile = blockIdx.x / p.k_split;
  const int split = blockIdx.x - tile * p.k_split;
  const int bidx = blockIdx.y;
  const int n0 = tile * NB;
  const int M = p.M, N = p.N, K = p.K;
  const int kbeg = split * p.k_chunk;
  const int klen = min(p.k_chunk, K - kbeg);   // > 0 by construction
  const int T = (klen + 63) / 64;

  const int8_t *Ab = p.A + bidx * p.sa;
  const int8_t *Bb = p.B + bidx * p.sb;

  // B slice addressing (row-major [64][NB] per slice).
  int b_row[CB], b_col[CB], b_lds[CB];
#pragma unroll
  for (int i = 0; i < CB; ++i) {
    const int row = tid / BCH + (256 / BCH) * i, c = tid % BCH;
    b_row[i] = row;
    b_col[i] = min(n0 + c * 16, N - 16);
    b_lds[i] = row * NB + ((c ^ b_swz<BCH>(row)) << 4);
  }
  v4i rb[U][CB];
  auto load_slice = [&](int s, v4i *dst) {
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      const int krow = min(kbeg + s * 64 + b_row[i], K - 1);
      dst[i] = *(const v4i *)(Bb + (int64_t)krow * p.ldb + b_col[i]);
    }
  };
  // Put the first U slices in flight before touching A.
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (u < T) load_slice(u, rb[u]);

  // A slice -> LDS, [16][k_chunk] with zero rows past M and zero k past K.
  {
    const int cpr = p.k_chunk / 16;   // chunks per row
    for (int i = tid; i < 16 * cpr; i += 256) {
      const int row = i / cpr, c = i - row * cpr;
      const int k = kbeg + c * 16;
      v4i v = v4i{0, 0, 0, 0};
      if (row < M && k < K) v = *(const v4i *)(Ab + (int64_t)row * p.lda + k);
      st_lds_b128(As, row * a_stride + c * 16, v);
    }
  }

  const int g = lane >> 4, j = lane & 15;
  int b_frag[NBW];
#pragma unroll
  for (int nb = 0; nb < NBW; ++nb) {
    const int cc = wave * NBW + nb;
    const int r0 = g * 16 + (j >> 1);
    b_frag[nb] = r0 * NB + ((cc ^ b_swz<BCH>(r0)) << 4) + (j & 1) * 8;
  }
  const int a_frag = (lane & 15) * a_stride + g * 16;

  v4i acc[NBW];
#pragma unroll
  for (int nb = 0; nb < NBW; ++nb) acc[nb] = v4i{0, 0, 0, 0};

  for (int t0 = 0; t0 < T; t0 += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = t0 + u;
      if (s < T) {
        int8_t *const Bs = Bs0 + (s & 1) * (64 * NB);
#pragma unroll
        for (int i = 0; i < CB; ++i) st_lds_b128(Bs, b_lds[i], rb[u][i]);
        if (s + U < T) load_slice(s + U, rb[u]);
        lds_barrier();
        const v4i a = ld_lds_b128(As, a_frag + s * 64);
#pragma unroll
        for (int nb = 0; nb < NBW; ++nb) {
          const v2i lo = ld_lds_tr8(Bs, b_frag[nb]);
          const v2i hi = ld_lds_tr8(Bs, b_frag[nb] + 8 * NB);
          const v4i b = v4i{lo.x, lo.y, hi.x, hi.y};
          acc[nb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[nb], 0, 0, 0);
        }
      }
    }
  }

  // 16x16 accumulator layout: element e of lane l is row 4*(l/16) + e,
  // column l%16.
  const int32_t *Db = HAS_D ? p.D + bidx * p.sd : nullptr;
  int32_t *Cb = p.C + bidx * p.sc;
  if (p.k_split == 1) {
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb) {
      const int col = n0 + (wave * NBW + nb) * 16 + j;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = g * 4 + e;
        if (row < M && col < N) {
          int32_t v = acc[nb][e];
          if (HAS_D) v = add_wrap(v, Db[(int64_t)row * p.ldd + col]);
          Cb[(int64_t)row * p.ldc + col] = v;
        }
      }
    }
    return;
  }

  // K split: publish this slice's partial, the last arriver reduces.
  int32_t *wsb = p.ws + (int64_t)bidx * p.k_split * 16 * N;
#pragma unroll
  for (int nb = 0; nb < NBW; ++nb) {
    const int col = n0 + (wave * NBW + nb) * 16 + j;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = g * 4 + e;
      if (row < M && col < N) wsb[((int64_t)split * 16 + row) * N + col] = acc[nb][e];
    }
  }
  __threadfence();
  __syncthreads();
  __shared__ int last;
  if (tid == 0) {
    int *ctr = p.counters + (int64_t)bidx * p.tiles_n + tile;
    const int prev = atomicAdd(ctr, 1);
    last = (prev == p.k_split - 1);
    if (last) *ctr = 0;   // every slice has arrived: reset for the next launch
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
#pragma unroll
  for (int nb = 0; nb < NBW; ++nb) {
    const int col = n0 + (wave * NBW + nb) * 16 + j;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = g * 4 + e;
      if (row < M && col < N) {
        int32_t v = HAS_D ? Db[(int64_t)row * p.ldd + col] : 0;
        for (int s = 0; s < p.k_split; ++s) {
          const int32_t part = (s == split)
              ? acc[nb][e]
              : wsb[((int64_t)s * 16 + row) * N + col];
          v = add_wrap(v, part);
        }
        Cb[(int64_t)row * p.ldc + col] = v;
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
      for (int64_t t = 0; t < p.K; ++t)
        s += (uint32_t)((int32_t)arow[t] * (int32_t)Bb[t * p.ldb + j]);
      p.C[b * p.sc + i * p.ldc + j] = (int32_t)s;
    }
  }
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

// lds_bytes of the skinny variants excludes the A slice (16 x (k_chunk+16)),
// which depends on K and the split.
const VariantInfo kVariants[VT_VARIANT_COUNT] = {
    {"auto", 0, 0, 0, 0, 0},
    {"mfma_256x256", 256, 256, 64, 256, 2 * (256 * 64 + 64 * 256)},
    {"mfma_128x128", 128, 128, 64, 256, 2 * (128 * 64 + 64 * 128)},
    {"skinny", 16, 128, 64, 256, 2 * 64 * 128},
    {"generic", 4, 64, 1, 256, 0},
    {"mfma_256x128", 256, 128, 64, 256, 2 * (256 * 64 + 64 * 128)},
};

constexpr int kSkinnyNB = 128;
constexpr int kMaxSkinnyLds = 160 * 1024 - 256;   // leave room for static LDS

struct Workspace {
  int32_t *partials = nullptr;
  size_t partial_bytes = 0;
  int *counters = nullptr;
  size_t counter_count = 0;
};

struct DeviceState {
  bool probed = false;
  bool ok = false;
  std::string arch;
  std::map<void *, Workspace> ws;   // per stream
};

std::mutex g_mu;
std::map<int, DeviceState> g_dev;

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
    st.ok = strncmp(prop.gcnArchName, "gfx950", 6) == 0;
    st.probed = true;
  }
  if (!st.ok)
    return fail(VT_ENODEV, "device %d is %s; this library is built for gfx950", dev,
                st.arch.c_str());
  *dev_out = dev;
  *st_out = &st;
  return VT_OK;
}

// Workspace for the skinny kernel's K split on (device, stream). Counters are
// zeroed once at allocation; each launch leaves them zero again.
int get_workspace(DeviceState *st, void *stream, size_t partial_bytes, size_t counters,
                  Workspace **out) {
  std::lock_guard<std::mutex> lk(g_mu);
  Workspace &w = st->ws[stream];
  if (w.partial_bytes < partial_bytes || w.counter_count < counters) {
    if (w.partials || w.counters) {
      VT_HIP_CHECK(hipStreamSynchronize((hipStream_t)stream));
      if (w.partials) VT_HIP_CHECK(hipFree(w.partials));
      if (w.counters) VT_HIP_CHECK(hipFree(w.counters));
      w = Workspace();
    }
    const size_t pb = partial_bytes > (1u << 20) ? partial_bytes : (1u << 20);
    const size_t cc = counters > 4096 ? counters : 4096;
    VT_HIP_CHECK(hipMalloc((void **)&w.partials, pb));
    VT_HIP_CHECK(hipMalloc((void **)&w.counters, cc * sizeof(int)));
    VT_HIP_CHECK(hipMemset(w.counters, 0, cc * sizeof(int)));
    w.partial_bytes = pb;
    w.counter_count = cc;
  }
  *out = &w;
  return VT_OK;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

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

int choose_k_split(int64_t N, int64_t K, int64_t batch) {
  const int64_t tiles = (N + kSkinnyNB - 1) / kSkinnyNB * batch;
  int64_t ks = (512 + tiles - 1) / tiles;     // aim for >= 2 workgroups per CU
  const int64_t max_by_k = K / 512 > 0 ? K / 512 : 1;   // slices >= 512 rows
  if (ks > max_by_k) ks = max_by_k;
  if (ks < 1) ks = 1;
  if (ks > 64) ks = 64;
  return (int)ks;
}

int select_variant(const Problem &q, bool vec, int32_t *variant, int32_t *k_split) {
  *k_split = 0;
  if (!vec || q.K == 0) {
    *variant = VT_VARIANT_GENERIC;
    return VT_OK;
  }
  if (q.M <= 16) {
    *variant = VT_VARIANT_SKINNY;
    *k_split = choose_k_split(q.N, q.K, q.batch);
    return VT_OK;
  }
  // Batched B-reuse with contiguous batches is one GEMM with stacked M.
  const bool fold = q.batch > 1 && q.sb == 0 && q.sa == q.M * q.lda && q.sc == q.M * q.ldc &&
                    (!q.D || q.sd == q.M * q.ldd);
  const int64_t m_eff = fold ? q.M * q.batch : q.M;
  const int64_t b_eff = fold ? 1 : q.batch;
  const int64_t t256 = (m_eff + 255) / 256 * ((q.N + 255) / 256) * b_eff;
  if (t256 >= 256 && q.N >= 256) {
    *variant = VT_VARIANT_MFMA_256x256;
  } else {
    const int64_t t128 = (m_eff + 255) / 256 * ((q.N + 127) / 128) * b_eff;
    *variant = (t128 >= 256 && m_eff >= 256) ? VT_VARIANT_MFMA_256x128
                                              : VT_VARIANT_MFMA_128x128;
  }
  return VT_OK;
}

template <int BM, int BN>
int launch_mfma(const Problem &q, hipStream_t stream) {
  // Fold contiguous shared-B batches into one stacked-M GEMM.
  Problem r = q;
  if (r.batch > 1 && r.sb == 0 && r.sa == r.M * r.lda && r.sc == r.M * r.ldc &&
      (!r.D || r.sd == r.M * r.ldd) && r.M * r.batch < (1ll << 30)) {
    r.M *= r.batch;
    r.batch = 1;
  }
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
  const bool edge = (r.M % BM) || (r.N % BN) || (r.K % 64);
  const bool has_d = r.D != nullptr;
  dim3 grid((unsigned)blocks), block(256);
  if (edge) {
    if (has_d) hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, true, true>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, true, false>), grid, block, 0, stream, a);
  } else {
    if (has_d) hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, false, true>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, false, false>), grid, block, 0, stream, a);
  }
  VT_HIP_CHECK(hipGetLastError());
  return VT_OK;
}

int launch_skinny(const Problem &q, int k_split, DeviceState *st, void *stream) {
  constexpr int NB = kSkinnyNB;
  if (q.M > 16) return fail(VT_EUNSUPPORTED, "skinny variant needs M <= 16 (M=%lld)", (long long)q.M);
  if (k_split <= 0) k_split = choose_k_split(q.N, q.K, q.batch);
  // Slice length: multiple of 64 rows; recompute the split count it implies.
  int64_t chunk = (q.K + k_split - 1) / k_split;
  chunk = (chunk + 63) / 64 * 64;
  int64_t lds = 16 * (chunk + 16) + 2 * 64 * NB;
  if (lds > kMaxSkinnyLds) {
    // Too long a slice for LDS: shrink it.
    chunk = ((kMaxSkinnyLds - 2 * 64 * NB) / 16 - 16) / 64 * 64;
    lds = 16 * (chunk + 16) + 2 * 64 * NB;
  }
  const int ks = (int)((q.K + chunk - 1) / chunk);
  SkinnyArgs a;
  a.A = q.A; a.B = q.B; a.D = q.D; a.C = q.C;
  a.lda = q.lda; a.ldb = q.ldb; a.ldd = q.ldd; a.ldc = q.ldc;
  a.sa = q.sa; a.sb = q.sb; a.sd = q.sd; a.sc = q.sc;
  a.M = (int)q.M; a.N = (int)q.N; a.K = (int)q.K;
  a.tiles_n = (int)((q.N + NB - 1) / NB);
  a.k_split = ks;
  a.k_chunk = (int)chunk;
  a.ws = nullptr;
  a.counters = nullptr;
  if ((int64_t)a.tiles_n * ks > 0x7fffffff || q.batch > 65535)
    return fail(VT_EUNSUPPORTED, "skinny grid too large");
  if (ks > 1) {
    Workspace *w = nullptr;
    const size_t pbytes = (size_t)q.batch * ks * 16 * q.N * sizeof(int32_t);
    const size_t nctr = (size_t)q.batch * a.tiles_n;
    int rc = get_workspace(st, stream, pbytes, nctr, &w);
    if (rc) return rc;
    a.ws = w->partials;
    a.counters = w->counters;
  }
  dim3 grid((unsigned)(a.tiles_n * ks), (unsigned)q.batch), block(256);
  // Allow dynamic LDS up to the per-CU size (once per kernel instantiation).
  static std::once_flag lds_attr_once;
  hipError_t attr_err = hipSuccess;
  std::call_once(lds_attr_once, [&] {
    hipError_t e1 = hipFuncSetAttribute((const void *)skinny_kernel<NB, true>,
                                        hipFuncAttributeMaxDynamicSharedMemorySize, kMaxSkinnyLds);
    hipError_t e2 = hipFuncSetAttribute((const void *)skinny_kernel<NB, false>,
                                        hipFuncAttributeMaxDynamicSharedMemorySize, kMaxSkinnyLds);
    attr_err = e1 != hipSuccess ? e1 : e2;
  });
  if (attr_err != hipSuccess)
    return fail(VT_EHIP, "hipFuncSetAttribute(skinny LDS) failed: %s", hipGetErrorString(attr_err));
  if (q.D)
    hipLaunchKernelGGL((skinny_kernel<NB, true>), grid, block, (size_t)lds, (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL((skinny_kernel<NB, false>), grid, block, (size_t)lds, (hipStream_t)stream, a);
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

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------

extern "C" {

int vt_abi_version(void) { return VT_ABI_VERSION; }

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
                   int32_t aligned, int32_t *variant_out, int32_t *k_split_out) {
  if (!variant_out || !k_split_out) return fail(VT_EINVAL, "null output pointer");
  if (M < 0 || N < 0 || K < 0 || batch < 0) return fail(VT_EINVAL, "negative size");
  Problem q = {};
  q.M = M; q.N = N; q.K = K; q.batch = batch; q.lda = lda; q.ldb = ldb;
  q.sa = M * lda; q.sb = 0; q.sc = M * N; q.ldc = N;
  const bool vec = aligned && q.N % 16 == 0 && q.K % 16 == 0 && q.K > 0 && lda % 16 == 0 &&
                   ldb % 16 == 0;
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
  // ---- host-side validation (never reaches the device on failure) ----
  if (M < 0 || N < 0 || K < 0 || batch < 0)
    return fail(VT_EINVAL, "negative size (M=%lld N=%lld K=%lld batch=%lld)", (long long)M,
                (long long)N, (long long)K, (long long)batch);
  if (variant < 0 || variant >= VT_VARIANT_COUNT)
    return fail(VT_EINVAL, "unknown variant %d", (int)variant);
  if (k_split < 0 || k_split > 4096) return fail(VT_EINVAL, "k_split %d out of range", (int)k_split);
  if (stride_a < 0 || stride_b < 0 || stride_d < 0 || stride_c < 0)
    return fail(VT_EINVAL, "negative batch stride");
  if (M == 0 || N == 0 || batch == 0) return VT_OK;
  if (!C) return fail(VT_EINVAL, "C is null");
  if (K > 0 && (!A || !B)) return fail(VT_EINVAL, "A or B is null");
  if (ldc < N) return fail(VT_EINVAL, "ldc=%lld < N=%lld", (long long)ldc, (long long)N);
  if (K > 0 && lda < K) return fail(VT_EINVAL, "lda=%lld < K=%lld", (long long)lda, (long long)K);
  if (K > 0 && ldb < N) return fail(VT_EINVAL, "ldb=%lld < N=%lld", (long long)ldb, (long long)N);
  if (D && ldd < N) return fail(VT_EINVAL, "ldd=%lld < N=%lld", (long long)ldd, (long long)N);
  if (batch > 1 && (stride_c < M * ldc && stride_c != 0))
    return fail(VT_EINVAL, "stride_c=%lld overlaps batches (M*ldc=%lld)", (long long)stride_c,
                (long long)(M * ldc));
  if (batch > 1 && stride_c == 0) return fail(VT_EINVAL, "stride_c must be nonzero for batch > 1");
  if (M > (1ll << 40) || N > (1ll << 40) || K > (1ll << 40))
    return fail(VT_EINVAL, "size beyond 2^40");

  Problem q = {A, B, D, C, M, N, K, lda, ldb, ldd, ldc, batch,
               stride_a, stride_b, stride_d, stride_c};
  const bool vec = vector_ok(q);
  int32_t chosen = variant, ks = k_split;
  if (variant == VT_VARIANT_AUTO) {
    select_variant(q, vec, &chosen, &ks);
    if (k_split > 0) ks = k_split;
  } else if (variant != VT_VARIANT_GENERIC) {
    if (!vec)
      return fail(VT_EUNSUPPORTED,
                  "variant %s needs N%%16==0, K%%16==0 (K>0), lda/ldb/strides multiples of 16 "
                  "and 16-byte aligned A, B",
                  kVariants[variant].name);
    if (variant == VT_VARIANT_SKINNY && M > 16)
      return fail(VT_EUNSUPPORTED, "variant skinny needs M <= 16 (M=%lld)", (long long)M);
  }
  if (chosen != VT_VARIANT_GENERIC && !vec)
    return fail(VT_EUNSUPPORTED, "internal: vector variant selected for an unaligned problem");

  int dev = 0;
  DeviceState *st = nullptr;
  int rc = current_device(&dev, &st);
  if (rc) return rc;
  hipStream_t s = (hipStream_t)stream;
  switch (chosen) {
    case VT_VARIANT_MFMA_256x256: return launch_mfma<256, 256>(q, s);
    case VT_VARIANT_MFMA_128x128: return launch_mfma<128, 128>(q, s);
    case VT_VARIANT_MFMA_256x128: return launch_mfma<256, 128>(q, s);
    case VT_VARIANT_SKINNY: return launch_skinny(q, ks, st, stream);
    case VT_VARIANT_GENERIC: return launch_generic(q, s);
    default: return fail(VT_EINVAL, "unknown variant %d", (int)chosen);
  }
}

}  // extern "C"
