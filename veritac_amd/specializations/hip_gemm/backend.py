"""hip_gemm backend: plans, validation, candidates and execution of the exact
int8 x int8 -> int32 GEMM on MI355X (gfx950).

Same verbs and conventions as the reference's Gemmini backend
(specializations/gemmini_gemm/backend.py):

  make_plan / required_resources / validate_plan   backend.py:1064, :97, :107
  gen_candidates / modeled_counts / modeled_objective / optimize
                                                   backend.py:336, :346, :370, :1072
  run (raises HipGemmError like run_commands raises GemminiError)
                                                   backend.py:380, :433-562

Conventions kept from the reference:
  * validate_plan returns (ok, reason) and never raises on bad input;
  * execution fails closed: an invalid plan, mismatched operands, a missing
    native library or no gfx950 device raise HipGemmError -- there is no CPU
    fallback;
  * the native library path can be overridden with VT_HIP_GEMM_LIB
    (cf. VERITAC_GEMMINI_CHECK_BIN, backend.py:156-161);
  * modeled counts are analytic models for candidate ranking, never
    measurements (backend.py:46-49).

Plan schema (all ints strict, bools strict):
  {"m", "n", "k", "batch", "dim", "b_shared", "has_d", "d_max_abs",
   "variant", "k_split"}
The contract extends the reference's full-tile DIM=16 GEMM: m may be any
positive size (the decode shapes have m = 1), n and k must be multiples of
DIM for the MFMA and skinny variants, and the overflow bound is
k*16384 + d_max_abs <= 2^31-1 (Plan.lean:86-92 plus the initial partial sum).
"""
from __future__ import annotations

import hashlib
import math

from ... import _lib
from ..._lib import HipGemmError

DIM = 16
ELEM_MIN, ELEM_MAX = -128, 127
ACC_ELEMENT_MAX = 2**31 - 1
INT8_DOMAIN_CONSTRAINT = "inputs are int8 in [-128,127] and k*16384 + |D| <= 2147483647"
MAX_EXTENT = 2**40

VARIANTS = ("mfma_256x256", "mfma_256x128", "mfma_128x128", "skinny", "generic", "padded")
# variants that take any n and k (no multiple-of-16 rule)
ANY_SHAPE_VARIANTS = ("generic", "padded")
# The packed-B decode variant takes B prepacked by pack_b (vt_pack_b_i8), not
# row-major, so it is never an automatic candidate for a row-major B.
PACKED_VARIANT = "skinny_packed"
ALL_VARIANTS = VARIANTS + (PACKED_VARIANT,)
SUPPORTED_VARIANTS = ("auto",) + ALL_VARIANTS

# variant -> (tile_m, tile_n, tile_k, threads, lds_bytes); mirrors the native
# table returned by vt_variant_info (checked by the tests).
# The MFMA variants' LDS is their tile kernel's: three 64-deep slice buffers.
TILES = {
    "mfma_256x256": (256, 256, 64, 256, 3 * (256 * 64 + 64 * 256)),
    "mfma_256x128": (256, 128, 64, 256, 3 * (256 * 64 + 64 * 128)),
    "mfma_128x128": (128, 128, 64, 256, 3 * (128 * 64 + 64 * 128)),
    "skinny": (16, 256, 64, 1024, 2 * 16 * 1024),
    "generic": (4, 64, 1, 256, 0),
    # padding granularity: A and B copied with k and n rounded up to 16, the
    # product run on the vector kernel the native selection picks for that shape
    "padded": (16, 16, 16, 256, 0),
    # up to 64 rows (groups of 64 for larger m), 4 column blocks, 64-row
    # blocks, 8 waves, LDS for the cross-wave sums (kPacked* in the HIP source)
    "skinny_packed": (64, 64, 64, 512, 8 * 4 * 1024),
}
PACKED_WAVES = 8
# LDS of the persistent 256x256 kernels, one workgroup per CU (kDmaLds and
# kDma16Lds in the HIP source): 4 slice stages, plus the 16x16x64 kernel's
# four 8 KiB epilogue strips. The 16x16x64 kernel runs K % 256 == 0.
DMA_LDS = 4 * (256 * 64 + 64 * 256)
DMA16_LDS = DMA_LDS + 4 * 8192
# An mfma_128x128 launch with row-major B runs 64x128 tiles, with this LDS
# per workgroup, when those tiles and the K split they call for give at most
# MFMA_HALF_MAX_WGS workgroups, each over at most MFMA_HALF_MAX_K of K
# (MFMA_HALF_MAX_SLICE_K per slice when K is split) (kHalfTile* in the HIP
# source).
MFMA_HALF_MAX_WGS, MFMA_HALF_MAX_K, MFMA_HALF_MAX_SLICE_K = 256, 2048, 1024
HALF_TILE_LDS = 3 * (64 * 64 + 64 * 128)
QUARTER_TILE_LDS = 3 * (64 * 64 + 64 * 64)
SKINNY_MAX_M = 64   # up to 4 row blocks of 16 (kSkinnyMaxM in the HIP source)
# Up to this many rows vt_gemm_i8 finishes a K-split skinny launch inside the
# kernel, through one 64-bit finishing word per two outputs (kSkinnyFinMaxM)
SKINNY_FIN_MAX_M = 16
# A slice's biased partial lies in [0, FIN_SPAN_PER_ROW * k_chunk]
# (kFinSpanPerRow: an int8 product lies in [-128 * 127, (-128)^2]).
FIN_SPAN_PER_ROW = 16256 + 16384
SKINNY_PIPE_ROWS = 64 * 2   # stage rows x stages in flight (kSkinny* in the HIP source)
LDS_PER_CU = 160 * 1024

# MI355X datasheet figures used by the analytic model and the rooflines.
PEAK_INT8_OPS = 256 * 2.4e9 * 8192      # dense INT8 MFMA, ops/s (~5.03e15)
PEAK_HBM_BYTES = 8.0e12                 # HBM3E, bytes/s
NUM_CUS = 256

_INT_FIELDS = ("m", "n", "k", "batch", "dim", "d_max_abs", "k_split")
_BOOL_FIELDS = ("b_shared", "has_d")


def _is_int(v):
    return isinstance(v, int) and not isinstance(v, bool)


# ---------------------------------------------------------------------------
# Plans
# ---------------------------------------------------------------------------

def skinny_split(plan):
    """(k_split, k_chunk) the skinny kernel launches for this plan.

    Mirrors launch_skinny_cfg in csrc/vt_hip_gemm.hip: the requested split (or
    the automatic one) becomes slices of a whole number of pipelines
    (SKINNY_PIPE_ROWS rows) whose A part fits in LDS.
    """
    k, ks = plan["k"], plan["k_split"]
    if ks <= 0:
        ks = _auto_k_split(plan["n"], k, plan["batch"])
    align = SKINNY_PIPE_ROWS
    stage_lds = TILES["skinny"][4]
    a_rows = 16 * skinny_row_blocks(plan["m"])
    chunk = -(-k // ks)
    chunk = -(-chunk // align) * align
    if a_rows * skinny_a_stride(chunk) + stage_lds > LDS_PER_CU:
        chunk = ((LDS_PER_CU - stage_lds) // a_rows - 48) // align * align
    return -(-k // chunk), chunk


def skinny_fin_bits(ks, chunk):
    """Width of each of the two sum fields of a finishing word for ks slices
    of chunk rows, or 0 when the arrival count no longer fits beside them
    (skinny_fin_bits in the HIP source)."""
    bits = (ks * chunk * FIN_SPAN_PER_ROW).bit_length()
    return bits if 2 * bits + (ks - 1).bit_length() <= 64 else 0


def skinny_finishes(plan):
    """Whether vt_gemm_i8 finishes this skinny plan's K slices inside the
    kernel (one launch) rather than in skinny_reduce_kernel (a second
    launch): a K split over at most SKINNY_FIN_MAX_M rows whose finishing
    word fits (skinny_finishes in the HIP source; vt_gemm_i8_noalloc always
    takes the second launch)."""
    ks, chunk = skinny_split(plan)
    return ks > 1 and plan["m"] <= SKINNY_FIN_MAX_M and skinny_fin_bits(ks, chunk) > 0


def packed_finishes(plan):
    """Whether the packed decode kernel finishes a packed plan's K slices
    inside the kernel (one launch) on the skinny kernel's terms: a K split
    over at most SKINNY_FIN_MAX_M rows whose finishing word fits (the
    packed launch in the HIP source; vt_gemm_i8_noalloc keeps the second
    launch)."""
    ks, per = packed_split(plan)
    return ks > 1 and plan["m"] <= SKINNY_FIN_MAX_M and skinny_fin_bits(ks, per * 64) > 0


def skinny_row_blocks(m):
    """Row blocks of 16 the skinny kernel runs for m rows: 1, 2 or 4
    (skinny_row_blocks in the HIP source)."""
    return 1 if m <= 16 else 2 if m <= 32 else 4


def skinny_a_stride(k_chunk):
    """LDS row pitch of the skinny kernel's A slice (skinny_a_stride in the
    HIP source): k_chunk padded to 2 (mod 4) 16-byte chunks."""
    return k_chunk + 16 * ((2 - (k_chunk >> 4)) & 3)


def _auto_k_split(n, k, batch):
    tiles = -(-n // TILES["skinny"][1]) * batch
    if tiles >= 192:
        return 1
    ks = -(-224 // tiles)
    ks = min(ks, -(-k // SKINNY_PIPE_ROWS))
    return max(1, min(ks, 64))


PACKED_NBW = 4   # 16-column blocks one packed workgroup holds


def packed_columns(plan, num_cus=NUM_CUS):
    """(8-column half blocks per column group, column groups per batch) of the
    packed kernel: whole groups of PACKED_NBW blocks when they give 192 or
    more workgroups, else groups as small as one per CU needs (down to half a
    block) instead of a K split. Mirrors packed_hpw / launch_packed_rows in
    csrc/vt_hip_gemm.hip, which use the device's CU count (256 on an MI355X)."""
    nbt, batch = plan["n"] // 16, plan["batch"]
    if -(-nbt // PACKED_NBW) * batch >= 192:
        hpw = 2 * PACKED_NBW
    else:
        hpw = max(1, min(-(-2 * nbt * batch // num_cus), 2 * PACKED_NBW))
    return hpw, -(-2 * nbt // hpw)


def packed_split(plan):
    """(k_split, 64-row blocks per slice) the packed kernel launches.

    Mirrors packed_k_split / launch_packed_rows in csrc/vt_hip_gemm.hip.
    """
    k, batch, ks = plan["k"], plan["batch"], plan["k_split"]
    kbt = -(-k // 64)
    if ks <= 0:
        groups = packed_columns(plan)[1] * batch
        if groups >= 192:
            ks = 1
        else:
            ks = max(1, min(-(-224 // groups), -(-kbt // PACKED_WAVES), 64))
    per = -(-kbt // ks)
    return -(-kbt // per), per


def _folded(plan):
    """(m, batch) with contiguous shared-B batches folded into m (mfma_fold)."""
    m, b = plan["m"], plan["batch"]
    return (m * b, 1) if plan["b_shared"] and b > 1 else (m, b)


def _k_split_for_tiles(m, n, k, b, tm, tn):
    """mfma_k_split<tm, tn> in the HIP source, on a folded problem: a k of at
    least 1024 over at most 64 tiles is cut into up to 16 slices of whole
    128-deep steps, each at least 512 deep, for up to 256 workgroups; from
    k = 8192 on, one over 65..128 tiles into two slices."""
    if b != 1 or k < 1024 or n % 16:
        return 1
    tiles = -(-m // tm) * -(-n // tn)
    if tiles * 4 > NUM_CUS:
        return 2 if tiles * 2 <= NUM_CUS and k >= 8192 and k % 256 == 0 else 1
    ks = 1
    while ks < 16 and 2 * ks * tiles <= NUM_CUS:
        ks *= 2
    while ks > 1 and (k % (128 * ks) or k // ks < 512):
        ks //= 2
    return ks


def mfma_k_split(plan):
    """K slices vt_gemm_i8 runs an MFMA plan in (mfma_split_for in the HIP
    source): a k of at least 1024 over at most 64 of the tiles the plan runs
    (contiguous shared-B batches folded into m) is cut into up to 16 slices of
    whole 128-deep steps, each at least 512 deep, for up to 256 workgroups
    (from k = 8192, into two over 65..128 tiles); the partial sums are added
    by a second kernel. 1: no split."""
    variant = plan["variant"]
    if not variant.startswith("mfma"):
        return 1
    tm, tn = mfma_tile_shape(plan)
    m, b = _folded(plan)
    return _k_split_for_tiles(m, plan["n"], plan["k"], b, tm, tn)


def mfma_split_rows(plan):
    """Rows of an mfma_256x256 plan (contiguous shared-B batches folded into
    m) that vt_gemm_i8 runs on the persistent 256x256 kernel before the rest
    run on 128x128 tiles (mfma_split_rows in the HIP source): the whole
    256-row tiles, when n is whole tiles and the last, partial tile row would
    add a round of tiles on 256 CUs. 0: one launch, whose last tile row, when
    partial, is moved back to end at m."""
    if plan["variant"] != "mfma_256x256":
        return 0
    m, n, k, b = plan["m"], plan["n"], plan["k"], plan["batch"]
    if plan["b_shared"] and b > 1:
        m, b = m * b, 1
    if m < 256 or m % 256 == 0 or n % 256 or k == 0 or k % 64:
        return 0
    row_tiles = n // 256 * b
    full = m // 256 * row_tiles
    return m // 256 * 256 if -(-(full + row_tiles) // NUM_CUS) > -(-full // NUM_CUS) else 0


def mfma_split_cols(plan):
    """The same for columns (mfma_split_cols in the HIP source): the whole
    256-column tiles of an mfma_256x256 plan run first when m is whole tiles
    and the last, partial tile column would add a round of tiles on 256 CUs;
    the other columns then run on 128x128 tiles. 0: no column split."""
    if plan["variant"] != "mfma_256x256":
        return 0
    m, n, k, b = plan["m"], plan["n"], plan["k"], plan["batch"]
    if plan["b_shared"] and b > 1:
        m, b = m * b, 1
    if n < 256 or n % 256 == 0 or m % 256 or k == 0 or k % 64:
        return 0
    col_tiles = m // 256 * b
    full = n // 256 * col_tiles
    return n // 256 * 256 if -(-(full + col_tiles) // NUM_CUS) > -(-full // NUM_CUS) else 0


def _mfma_parts(plan):
    """(the whole rows or columns on the persistent 256x256 kernel, the rest
    on 128x128 tiles) as two plans, or None when neither mfma_split_rows nor
    mfma_split_cols splits the plan."""
    rows = mfma_split_rows(plan)
    cols = 0 if rows else mfma_split_cols(plan)
    if not rows and not cols:
        return None
    if plan["b_shared"] and plan["batch"] > 1:
        plan = dict(plan, m=plan["m"] * plan["batch"], batch=1)
    if rows:
        top = dict(plan, m=rows, k_split=0)
        rest = dict(plan, m=plan["m"] - rows, variant="mfma_128x128", k_split=0)
    else:
        top = dict(plan, n=cols, k_split=0)
        rest = dict(plan, n=plan["n"] - cols, variant="mfma_128x128", k_split=0)
    return top, rest


PACKED_DMA_MIN_TILES = 128   # kPackedDmaMinTiles in the HIP source


def packed_dma_rows(plan):
    """Rows of a skinny_packed plan that run on the 256x256 MFMA kernel, when
    n % 256 == 0, k % 64 == 0, there are at least PACKED_DMA_MIN_TILES whole
    256-row tiles over all batches, and every lane offset from a tile's base
    fits 32 bits (contiguous A: 256 * k; packed B: 16 column blocks of kbt
    1 KiB tiles): all m rows (a partial last tile row is moved back to end at
    m, its stores masked), unless that partial row would add a round of tiles
    on 256 CUs, then the whole 256-row tiles. Mirrors packed_dma_rows in
    csrc/vt_hip_gemm.hip."""
    m, n, k, batch = plan["m"], plan["n"], plan["k"], plan["batch"]
    kbt = -(-k // 64)
    if not (m >= 256 and n % 256 == 0 and k % 64 == 0 and k > 0 and 256 * k < 2**32 - 4096
            and 16 * 1024 * kbt < 2**32 - 4096):
        return 0
    row_tiles = n // 256 * batch
    full = m // 256 * row_tiles
    if full < PACKED_DMA_MIN_TILES:
        return 0
    if m % 256 == 0 or -(-(full + row_tiles) // NUM_CUS) == -(-full // NUM_CUS):
        return m
    return m // 256 * 256


def packed_tiles_fit(plan):
    """Whether packed rows can run on 128x128 MFMA tiles: lane offsets from a
    tile's base within 32 bits (contiguous A: 256 * k; packed B: 8 column
    blocks of kbt 1 KiB tiles). packed_tiles_fit in the HIP source."""
    k = plan["k"]
    return 256 * k < 2**32 - 4096 and 8 * 1024 * -(-k // 64) < 2**32 - 4096


def packed_dma128(plan):
    """Whether a skinny_packed plan runs whole on the persistent kernel's
    256x128 form (packed_dma128_fits in the HIP source): no rows on the
    256x256 kernel, m >= 256, n % 128 == 0, k % 256 == 0, k >= 1024, lane
    offsets within 32 bits, and more than 128 but at most 256 tiles of
    256x128 over all batches."""
    m, n, k, batch = plan["m"], plan["n"], plan["k"], plan["batch"]
    if packed_dma_rows(plan) or not (m >= 256 and n % 128 == 0 and k % 256 == 0 and k >= 1024):
        return False
    if not (256 * k < 2**32 - 4096 and 8 * 1024 * (k // 64) < 2**32 - 4096):
        return False
    return 128 < -(-m // 256) * (n // 128) * batch <= 256


def _packed_parts(plan):
    """(plan of the rows on the persistent kernel or None, plan of the other
    rows or None) of a skinny_packed plan: rows on the 256x256 kernel, or all
    of them on its 256x128 form (variant mfma_256x128). More than
    SKINNY_MAX_M other rows run as 128x128 MFMA tiles (variant mfma_128x128);
    up to that many, in one group on the packed decode kernel (variant
    skinny_packed)."""
    if packed_dma128(plan):
        return dict(plan, variant="mfma_256x128", k_split=0, b_shared=False, packed_b=True), None
    rows = packed_dma_rows(plan)
    dma = dict(plan, m=rows, variant="mfma_256x256", k_split=0) if rows else None
    rest = None
    if plan["m"] > rows:
        rest = dict(plan, m=plan["m"] - rows)
        if rest["m"] > SKINNY_MAX_M and packed_tiles_fit(plan):
            # after the 256-row tiles the batches are no longer contiguous
            # blocks of rows, so the library does not fold them into one GEMM
            rest = dict(rest, variant="mfma_128x128", k_split=0,
                        b_shared=plan["b_shared"] and not rows, packed_b=True)
    return dma, rest


def persistent_lds(k):
    """LDS per workgroup of the persistent 256x256 kernel for a K (slice):
    the 16x16x64 kernel when K % 256 == 0, else the 32x32x32 one (plans
    assume 16-byte aligned C and D with rows of n elements)."""
    return DMA16_LDS if k % 256 == 0 else DMA_LDS


def mfma_half_tiles(plan):
    """Whether an mfma_128x128 plan runs 64x128 tiles (mfma_half_rows in the
    HIP source): row-major B, and 64x128 tiles with the K split they call for
    give at most MFMA_HALF_MAX_WGS workgroups, each over at most
    MFMA_HALF_MAX_K of K, or MFMA_HALF_MAX_SLICE_K per slice when K is split
    (shared-B batches folded)."""
    if plan["variant"] != "mfma_128x128" or plan.get("packed_b"):
        return False
    m, b = _folded(plan)
    n, k = plan["n"], plan["k"]
    ks = _k_split_for_tiles(m, n, k, b, 64, 128)
    return (-(-m // 64) * -(-n // 128) * b * ks <= MFMA_HALF_MAX_WGS and
            k // ks <= (MFMA_HALF_MAX_SLICE_K if ks > 1 else MFMA_HALF_MAX_K))


def mfma_quarter_tiles(plan):
    """Whether an mfma_128x128 plan runs 64x64 tiles (mfma_quarter_tiles in
    the HIP source): it runs 64x128 tiles, and 64x64 tiles with their own K
    split also give at most MFMA_HALF_MAX_WGS workgroups, each over at most
    MFMA_HALF_MAX_K of K (MFMA_HALF_MAX_SLICE_K per slice when split)."""
    if not mfma_half_tiles(plan):
        return False
    m, b = _folded(plan)
    n, k = plan["n"], plan["k"]
    ks = _k_split_for_tiles(m, n, k, b, 64, 64)
    return (-(-m // 64) * -(-n // 64) * b * ks <= MFMA_HALF_MAX_WGS and
            k // ks <= (MFMA_HALF_MAX_SLICE_K if ks > 1 else MFMA_HALF_MAX_K))


def mfma_tile_shape(plan):
    """(rows, columns) of the output tiles an MFMA plan's kernel runs."""
    tm, tn = TILES[plan["variant"]][:2]
    if mfma_quarter_tiles(plan):
        return 64, 64
    return (64 if mfma_half_tiles(plan) else tm), tn


def mfma_tiles(plan):
    """Output tiles an MFMA plan runs, over every batch and K slice (shared-B
    batches folded into m); the persistent kernel walks them in rounds."""
    tm, tn = mfma_tile_shape(plan)
    m, batch = plan["m"], plan["batch"]
    if plan["b_shared"] and batch > 1:
        m, batch = m * batch, 1
    return -(-m // tm) * -(-plan["n"] // tn) * batch * mfma_k_split(plan)


def _runs_persistent(plan):
    """Whether an mfma_256x256 plan (without a row or column split) runs on
    the persistent kernel: each K slice in whole 64-deep steps and M (after
    the fold) and N at least one tile (persistent_fits in the HIP source).
    An mfma_256x128 plan runs on the persistent kernel's 256x128 form when M
    (after the fold) is at least 256, N at least 128 and each K slice whole
    256-deep groups (dma16_128_fits; plans assume 16-byte aligned C and D
    with rows of n elements)."""
    if plan["variant"] not in ("mfma_256x256", "mfma_256x128"):
        return False
    m = plan["m"] * plan["batch"] if plan["b_shared"] and plan["batch"] > 1 else plan["m"]
    kslice = plan["k"] // mfma_k_split(plan)
    if plan["variant"] == "mfma_256x128":
        return kslice > 0 and kslice % 256 == 0 and m >= 256 and plan["n"] >= 128
    return kslice > 0 and kslice % 64 == 0 and m >= 256 and plan["n"] >= 256


def required_resources(plan):
    """(lds_bytes per workgroup, workgroups) the plan's variant launches.

    The analogue of backend.py:97-104 (scratchpad / accumulator rows) for a
    gfx950 launch: LDS is the on-chip buffer a workgroup needs, workgroups
    the grid size. The persistent 256x256 kernel launches one workgroup per
    CU (at most) whatever the tile count, and so does its 256x128 form.
    """
    variant = plan["variant"]
    tm, tn, _, _, lds = TILES[variant]
    m, n, batch = plan["m"], plan["n"], plan["batch"]
    if variant.startswith("mfma"):
        parts = _mfma_parts(plan)
        if parts is not None:   # whole tiles on the persistent kernel, then the rest
            top, rest = parts
            lds_t, wgs_t = required_resources(top)
            lds_r, wgs_r = required_resources(rest)
            return max(lds_t, lds_r), wgs_t + wgs_r
        if _runs_persistent(plan):
            return persistent_lds(plan["k"] // mfma_k_split(plan)), min(mfma_tiles(plan), NUM_CUS)
        shape = mfma_tile_shape(plan)
        return ({(64, 64): QUARTER_TILE_LDS, (64, 128): HALF_TILE_LDS}.get(shape, lds),
                mfma_tiles(plan))
    if variant == "skinny":
        ks, chunk = skinny_split(plan)
        return (lds + 16 * skinny_row_blocks(m) * skinny_a_stride(chunk),
                -(-n // tn) * ks * batch)
    if variant == PACKED_VARIANT:
        dma, rest = _packed_parts(plan)
        lds_out, wgs = 0, 0
        if dma is not None:
            lds_out, wgs = persistent_lds(plan["k"]), min(required_resources(dma)[1], NUM_CUS)
        if rest is not None and rest["variant"] != PACKED_VARIANT:
            lds_r, wgs_r = required_resources(rest)
            lds_out, wgs = max(lds_out, lds_r), wgs + wgs_r
        elif rest is not None:
            ks, _ = packed_split(rest)
            lds_out = max(lds_out, lds)
            wgs += packed_columns(rest)[1] * ks * batch * -(-rest["m"] // tm)
        return lds_out, wgs
    if variant == "padded":
        return required_resources(padded_inner_plan(plan))
    return 0, -(-n // tn) * min(-(-m // tm), 65535) * min(batch, 65535)


def padded_inner_plan(plan):
    """The plan the padded variant runs after copying A and B with k and n
    rounded up to 16: the vector variant the native selection picks for that
    shape (vt_gemm_select). D goes to the product when n is a multiple of 16
    (it writes C directly), else it is added while copying C out."""
    n_p, k_p = -(-plan["n"] // DIM) * DIM, -(-plan["k"] // DIM) * DIM
    name, ks = _lib.select_variant(plan["m"], n_p, k_p, plan["batch"], k_p, n_p, True,
                                   b_shared=plan["b_shared"])
    d = plan["has_d"] and n_p == plan["n"]
    return dict(plan, n=n_p, k=k_p, variant=name, k_split=ks, has_d=d,
                d_max_abs=plan["d_max_abs"] if d else 0)


def _padded_copies(plan):
    """(copy A, copy B, copy C out) for contiguous, 16-byte-aligned operands:
    an operand the vector kernels can read as it is is not copied."""
    k_odd, n_odd = plan["k"] % DIM != 0, plan["n"] % DIM != 0
    return k_odd, k_odd or n_odd, n_odd


def make_plan(m, n, k, *, batch=1, b_shared=False, has_d=False, d_max_abs=0,
              variant="auto", k_split=0):
    """A plan for C[batch] = D + A[batch].B; "auto" resolves the variant natively.

    Mirrors backend.py:1064-1069. variant="auto" asks the native library
    (vt_gemm_select) which kernel it would launch, so the plan records the
    concrete variant and K split.
    """
    plan = {"m": m, "n": n, "k": k, "batch": batch, "dim": DIM,
            "b_shared": bool(b_shared), "has_d": bool(has_d), "d_max_abs": d_max_abs,
            "variant": variant, "k_split": k_split}
    if variant == "auto":
        ok, reason = validate_plan(dict(plan, variant="generic"))
        if not ok:
            raise HipGemmError("cannot plan: " + reason)
        vec = n % DIM == 0 and k % DIM == 0
        name, ks = _lib.select_variant(m, n, k, batch, k, n, vec, b_shared=b_shared)
        plan["variant"] = name
        if name == "skinny" and k_split == 0:
            plan["k_split"] = ks
    return plan


def validate_plan(plan):
    """Structural, divisibility, overflow and resource validation -> (ok, reason).

    Mirrors backend.py:107-149: never raises, rejects bools and non-integers
    for integer fields, checks the overflow bound and the buffer extents.
    """
    if not isinstance(plan, dict):
        return False, "plan must be a JSON object"
    for key in _INT_FIELDS:
        if key not in plan or not _is_int(plan[key]):
            return False, "plan field %r must be an integer" % key
    for key in _BOOL_FIELDS:
        if key not in plan or not isinstance(plan[key], bool):
            return False, "plan field %r must be a boolean" % key
    variant = plan.get("variant")
    if variant not in ALL_VARIANTS:
        return False, ("unsupported variant %r (supported: %s)" % (variant, list(ALL_VARIANTS)))
    m, n, k, batch, dim = plan["m"], plan["n"], plan["k"], plan["batch"], plan["dim"]
    if dim != DIM:
        return False, "dim must equal DIM=%d (got %d)" % (DIM, dim)
    for name, val in (("m", m), ("n", n), ("k", k), ("batch", batch)):
        if val <= 0:
            return False, "%s=%d must be positive" % (name, val)
    if plan["d_max_abs"] < 0:
        return False, "d_max_abs must be >= 0"
    if not plan["has_d"] and plan["d_max_abs"] != 0:
        return False, "d_max_abs must be 0 without an initial partial sum"
    if plan["k_split"] < 0:
        return False, "k_split must be >= 0"
    bound = k * 16384 + plan["d_max_abs"]
    if bound > ACC_ELEMENT_MAX:
        return False, ("overflow bound violated: k*16384 + d_max_abs = %d > 2147483647 (%s)"
                       % (bound, INT8_DOMAIN_CONSTRAINT))
    if max(m, n, k) >= MAX_EXTENT or batch * max(m * n, m * k) >= 2**62:
        return False, "buffer extent exceeds the supported indexing range"
    if variant not in ANY_SHAPE_VARIANTS:
        for name, val in (("n", n), ("k", k)):
            if val % dim != 0:
                return False, ("%s=%d must be divisible by dim=%d for variant %r"
                               % (name, val, dim, variant))
    if variant == "skinny":
        if m > SKINNY_MAX_M:
            return False, "variant 'skinny' needs m <= %d (got %d)" % (SKINNY_MAX_M, m)
        if batch > 65535:
            return False, "variant 'skinny' supports batch <= 65535"
    elif variant == PACKED_VARIANT:
        if batch > 65535:
            return False, "variant %r supports batch <= 65535" % PACKED_VARIANT
        if max(m, n, k) >= 2**30:
            return False, "variant %r needs m, n, k < 2^30" % PACKED_VARIANT
    elif variant == "padded":
        if plan["k_split"] != 0:
            return False, "variant 'padded' chooses its own k_split (give 0)"
        if m >= 2**30 or n + 15 >= 2**30 or k + 15 >= 2**30 or batch > 65535:
            return False, "variant 'padded' needs m, n+15, k+15 < 2^30 and batch <= 65535"
    elif variant != "generic" and plan["k_split"] != 0:
        return False, "k_split applies to variants 'skinny' and %r only" % PACKED_VARIANT
    try:
        lds, workgroups = required_resources(plan)
    except HipGemmError as exc:
        # the padded variant's inner plan comes from the native selection
        return False, "cannot resolve the %r launch: %s (fail-closed)" % (variant, exc)
    if lds > LDS_PER_CU:
        return False, "LDS %d bytes > %d per CU" % (lds, LDS_PER_CU)
    if workgroups > 2**31 - 1:
        return False, "grid of %d workgroups exceeds the launch limit" % workgroups
    return True, "ok"


# ---------------------------------------------------------------------------
# Analytic model (NOT a measurement)
# ---------------------------------------------------------------------------

# Fraction of the dense INT8 peak each variant is modeled at when compute-bound.
_MODEL_MFMA_EFF = {"mfma_256x256": 0.70, "mfma_256x128": 0.60, "mfma_128x128": 0.45,
                   "skinny": 0.25, "skinny_packed": 0.25, "generic": 0.002}


def algorithmic_bytes(plan):
    """A once + B once (shared B counted once) + C written + D read."""
    m, n, k, b = plan["m"], plan["n"], plan["k"], plan["batch"]
    a_bytes = b * m * k
    b_bytes = k * n if (plan["b_shared"] or b == 1) else b * k * n
    c_bytes = 4 * b * m * n
    d_bytes = c_bytes if plan["has_d"] else 0
    return a_bytes + b_bytes + c_bytes + d_bytes


def modeled_counts(plan):
    """Analytic ops / bytes / workgroups for a valid plan (a model, not a measurement)."""
    m, n, k, b = plan["m"], plan["n"], plan["k"], plan["batch"]
    variant = plan["variant"]
    tm, tn = mfma_tile_shape(plan) if variant.startswith("mfma") else TILES[variant][:2]
    lds, wgs = required_resources(plan)
    ops = 2 * b * m * n * k
    alg = algorithmic_bytes(plan)
    parts = _mfma_parts(plan) if variant.startswith("mfma") else None
    if parts is not None:
        l2_bytes = sum(modeled_counts(p)["bytes_l2_modeled"] for p in parts)
    elif variant.startswith("mfma"):
        m_eff, b_eff = (m * b, 1) if (plan["b_shared"] and b > 1) else (m, b)
        tiles_m, tiles_n = -(-m_eff // tm), -(-n // tn)
        # every tile reads its A row-panel and B column-panel once
        c_and_d = 4 * b * m * n * (2 if plan["has_d"] else 1)
        ks = mfma_k_split(plan)
        partial = 2 * 4 * ks * m_eff * n if ks > 1 else 0   # written, then read back
        l2_bytes = b_eff * (tiles_n * m_eff * k + tiles_m * k * n) + c_and_d + partial
    elif variant == "skinny":
        ks, _ = skinny_split(plan)
        # partial sums written and read back, or each slice's atomic add on
        # an 8-byte finishing word per two rows (read and written where it
        # is performed)
        partial = (16 * b * -(-m // 2) * n * ks if skinny_finishes(plan) else
                   2 * 4 * b * m * n * ks if ks > 1 else 0)
        l2_bytes = alg + partial + b * -(-n // tn) * 16 * k
    elif variant == PACKED_VARIANT:
        dma, rest = _packed_parts(plan)
        l2_bytes = modeled_counts(dma)["bytes_l2_modeled"] if dma is not None else 0
        if rest is not None and rest["variant"] != PACKED_VARIANT:
            l2_bytes += modeled_counts(rest)["bytes_l2_modeled"]
        elif rest is not None:
            mr = rest["m"]
            ks, _ = packed_split(rest)
            groups = -(-mr // SKINNY_MAX_M)
            partial = (16 * b * -(-mr // 2) * n * ks if packed_finishes(rest) else
                       2 * 4 * b * mr * n * ks if ks > 1 else 0)
            # B once per group of up to 64 rows; each column group reads its A rows once
            l2_bytes += (groups * (b * -(-k // 64) * 64 * n) + b * mr * k * packed_columns(rest)[1]
                         + 4 * b * mr * n * (2 if plan["has_d"] else 1) + partial)
    elif variant == "padded":
        inner = padded_inner_plan(plan)
        l2_bytes = modeled_counts(inner)["bytes_l2_modeled"] + _padded_copy_bytes(plan, inner)
    else:
        l2_bytes = b * (m * n * k + -(-m // 4) * n * k) + 4 * b * m * n
    return {"ops": ops, "macs": ops // 2, "bytes_algorithmic": alg, "bytes_l2_modeled": l2_bytes,
            "workgroups": wgs, "lds_bytes": lds,
            "arithmetic_intensity": ops / alg if alg else math.inf}


def _padded_copy_bytes(plan, inner):
    """Bytes the padded variant moves besides its inner product: each copied
    operand read and its padded copy written, and, when C is copied out, C'
    read back and C written (plus D)."""
    m, n, k, b = plan["m"], plan["n"], plan["k"], plan["batch"]
    n_p, k_p = inner["n"], inner["k"]
    b_mats = 1 if plan["b_shared"] or b == 1 else b
    copy_a, copy_b, copy_c = _padded_copies(plan)
    return ((b * m * (k + k_p) if copy_a else 0) + (b_mats * (k * n + k_p * n_p) if copy_b else 0)
            + (4 * b * m * n_p + 4 * b * m * n * (2 if plan["has_d"] else 1) if copy_c else 0))


# Latency floors measured on an MI355X (seconds): one kernel launch in a HIP
# graph; one load -> MFMA -> store round trip of a vector kernel; one 64-deep
# K slice of an MFMA workgroup; 16 K steps of the VALU kernel (its loads of
# A and B are issued 16 at a time).
_LAUNCH_S = 1.6e-6
_ROUND_TRIP_S = 2.0e-6
_SLICE_S = 0.35e-6
_GENERIC_STEP_S = 0.3e-6


def modeled_objective(plan, counts):
    """(modeled seconds, workgroups); least is best. A model, not a measurement.

    Compute time prices the padded tile work (rows/columns a tile covers past
    m and n still run MFMAs) at a per-variant fraction of the dense INT8 peak
    with whole-chip wave quantisation; memory time prices the algorithmic
    bytes at the HBM peak scaled down when the grid has fewer workgroups than
    CUs to keep loads in flight.
    """
    m, n, k, b = plan["m"], plan["n"], plan["k"], plan["batch"]
    variant = plan["variant"]
    if variant == "padded":
        # the inner product's objective, plus the copies at the HBM rate and
        # their launches (one for the operands, one for the copy-out)
        inner = padded_inner_plan(plan)
        t_inner, wgs = modeled_objective(inner, modeled_counts(inner))
        copy_a, copy_b, copy_c = _padded_copies(plan)
        launches = int(copy_a or copy_b) + int(copy_c)
        return (t_inner + _padded_copy_bytes(plan, inner) / PEAK_HBM_BYTES + launches * _LAUNCH_S, wgs)
    if variant.startswith("mfma") and _mfma_parts(plan) is not None:
        # whole 256-row tiles on the persistent kernel, then 128x128 tiles
        t, wgs = 0.0, 0
        for part in _mfma_parts(plan):
            tp, wp = modeled_objective(part, modeled_counts(part))
            t, wgs = t + tp, wgs + wp
        return t, wgs
    if variant == PACKED_VARIANT:
        parts = [p for p in _packed_parts(plan) if p is not None]
        if any(p["variant"] != PACKED_VARIANT for p in parts):
            # 256-row tiles on the 256x256 kernel and / or 128x128 tiles, and
            # at most one group on the decode kernel: launches in sequence
            t, wgs = 0.0, 0
            for part in parts:
                tp, wp = modeled_objective(part, modeled_counts(part))
                t, wgs = t + tp, wgs + wp
            return t, wgs
    tm, tn = mfma_tile_shape(plan) if variant.startswith("mfma") else TILES[variant][:2]
    if variant.startswith("mfma") and plan["b_shared"] and b > 1:
        m, b = m * b, 1
    padded_ops = 2 * b * (-(-m // tm) * tm) * (-(-n // tn) * tn) * k
    wgs = counts["workgroups"]
    # rounds of work over the CUs: MFMA tiles (the persistent kernel walks
    # them with one workgroup per CU), else workgroups
    units = mfma_tiles(plan) if variant.startswith("mfma") else wgs
    waves = -(-units // NUM_CUS)
    fill = units / (waves * NUM_CUS) if units else 1.0
    eff = _MODEL_MFMA_EFF[variant] * (fill if variant.startswith("mfma") else 1.0)
    t_compute = padded_ops / (PEAK_INT8_OPS * eff)
    t_memory = counts["bytes_algorithmic"] / (PEAK_HBM_BYTES * min(1.0, wgs / NUM_CUS))
    t = max(t_compute, t_memory)
    # latency floors: a launch each, and a workgroup's K loop
    if variant == "generic":
        return (_LAUNCH_S + max(t, -(-k // 16) * _GENERIC_STEP_S), wgs)
    launches = 1
    if variant == "skinny":
        launches += skinny_split(plan)[0] > 1 and not skinny_finishes(plan)
    elif variant == PACKED_VARIANT:
        launches += packed_split(plan)[0] > 1 and not packed_finishes(plan)
    else:
        ks = mfma_k_split(plan)
        launches += ks > 1
        t = max(t, -(-(k // ks) // 64) * _SLICE_S)
    return (launches * _LAUNCH_S + _ROUND_TRIP_S + t, wgs)


def sha256_file(path):
    """Hex sha256 of a file's bytes (backend.py:605-610)."""
    h = hashlib.sha256()
    with open(path, "rb") as fh:
        for chunk in iter(lambda: fh.read(65536), b""):
            h.update(chunk)
    return h.hexdigest()


def emit_c(plan, out_path, *, seed=0x12345678, input_mode="lcg"):
    """Emit a standalone self-checking C program for the plan (backend.py:817-846):
    refuses invalid or natively rejected plans, returns {path, sha256, counts}.
    The program runs the GEMM through the C ABI on the GPU and prints
    VERITAC_HIP_GEMM_PASS only after every output matched its scalar loop
    (program.emit_c)."""
    from .program import emit_c as _emit_c
    return _emit_c(plan, out_path, seed=seed, input_mode=input_mode)


def native_check(plan):
    """The native library's verdict on a valid plan -> (accepted, reason).

    Asks vt_gemm_check whether vt_gemm_i8 accepts the plan's call on
    contiguous operands (the refusal reasons are the native ones). Fail-closed
    like the reference's external checker (backend.py:164-196): a library
    that is missing or cannot load, or a plan with no native counterpart,
    is a rejection, never an acceptance.
    """
    m, n, k, b = plan["m"], plan["n"], plan["k"], plan["batch"]
    if plan["variant"] == PACKED_VARIANT:
        if n % DIM or k % DIM:
            return False, "packed B needs n and k divisible by 16"
        try:
            _lib.packed_b_size(k, n)
        except HipGemmError as exc:
            return False, "%s (fail-closed)" % exc
        dma, rest = _packed_parts(plan)
        how = []
        if dma is not None:
            how.append("%d rows on the %s kernel" % (
                dma["m"], "256x256" if dma["variant"] == "mfma_256x256" else "256x128 persistent"))
        if rest is not None and rest["variant"] != PACKED_VARIANT:
            how.append("%d on 128x128 tiles" % rest["m"])
        elif rest is not None:
            how.append("%d in a group of up to 64" % rest["m"])
        how = ", ".join(how)
        return True, "accepted: vt_packed_b_size takes k=%d n=%d; runs skinny_packed (%s)" % (
            k, n, how)
    sb = 0 if (plan["b_shared"] or b == 1) else k * n
    multi = b > 1
    try:
        st, reason, variant, ks, ws = _lib.gemm_check(
            m, n, k, k, n, n, n, b, m * k if multi else 0, sb, m * n if multi else 0,
            m * n if multi else 0, plan["has_d"], plan["variant"], plan["k_split"])
    except HipGemmError as exc:
        return False, "native check unavailable: %s (fail-closed)" % exc
    if st != _lib.VT_OK:
        return False, "vt_gemm_check: %s (%s)" % (reason, _lib.STATUS_NAMES.get(st, st))
    if variant != plan["variant"] and plan["variant"] != "auto":
        return False, ("vt_gemm_check would run %r for a %r plan (fail-closed)"
                       % (variant, plan["variant"]))
    how = ""
    parts = _mfma_parts(dict(plan, variant=variant))
    if parts is not None and parts[0]["n"] == parts[1]["n"]:
        how = "; %d rows on the persistent 256x256 kernel, %d on 128x128 tiles" % (
            parts[0]["m"], parts[1]["m"])
    elif parts is not None:
        how = "; %d columns on the persistent 256x256 kernel, %d on 128x128 tiles" % (
            parts[0]["n"], parts[1]["n"])
    return True, "accepted by vt_gemm_check: runs %s (k_split %d, %d bytes of workspace%s)" % (
        variant, ks, ws, how)


def gen_candidates(m, n, k, *, batch=1, b_shared=False, has_d=False, d_max_abs=0):
    """One plan per variant (the reference's per-schedule plans, backend.py:1080-1082)."""
    return [make_plan(m, n, k, batch=batch, b_shared=b_shared, has_d=has_d,
                      d_max_abs=d_max_abs, variant=v) for v in VARIANTS]


def optimize(m, n, k, *, batch=1, b_shared=False, has_d=False, d_max_abs=0,
             measure=False, num_runs=10):
    """Validate every variant, score it, pick the least modeled (or measured) time.

    Mirrors backend.py:1072-1093: returns {"candidates": [...], "winner": plan}
    with one entry per variant {plan, valid, invalid_reason,
    check{accepted, reason}, counts, objective} (plus measured_ms). `check`
    is the native library's verdict (native_check, fail-closed); only
    candidates that are valid and accepted are scored and eligible. With
    measure=True the eligible candidates are also timed on the GPU
    (runner.benchmark_gemm) and the winner is the fastest one whose measured
    output was correct (measured_ms, measured_correct); the modeled
    objective is kept alongside.
    """
    candidates = []
    for plan in gen_candidates(m, n, k, batch=batch, b_shared=b_shared, has_d=has_d,
                               d_max_abs=d_max_abs):
        ok, reason = validate_plan(plan)
        if ok:
            accepted, chk_reason = native_check(plan)
        else:
            accepted, chk_reason = False, "not checked: plan invalid (%s)" % reason
        entry = {"plan": plan, "valid": ok, "invalid_reason": None if ok else reason,
                 "check": {"accepted": accepted, "reason": chk_reason},
                 "counts": None, "objective": None, "measured_ms": None,
                 "measured_correct": None}
        if ok and accepted:
            counts = modeled_counts(plan)
            entry["counts"] = counts
            entry["objective"] = modeled_objective(plan, counts)
        candidates.append(entry)
    eligible = [c for c in candidates if c["valid"] and c["check"]["accepted"]]
    if measure and eligible:
        from . import runner
        for c in eligible:
            res = runner.benchmark_gemm(c["plan"], num_runs=num_runs, warmup=2, rotate=False,
                                        cpu_budget_s=0.05)
            c["measured_ms"] = res["gpu_time_ms"]
            c["measured_correct"] = res["correct"]
        # a candidate whose measured output was wrong never wins
        correct = [c for c in eligible if c["measured_correct"]]
        winner = min(correct, key=lambda c: c["measured_ms"])["plan"] if correct else None
    else:
        winner = min(eligible, key=lambda c: c["objective"])["plan"] if eligible else None
    return {"candidates": candidates, "winner": winner}


# ---------------------------------------------------------------------------
# Execution
# ---------------------------------------------------------------------------

def _torch():
    import torch
    return torch


def _operand_shapes(plan):
    m, n, k, b = plan["m"], plan["n"], plan["k"], plan["batch"]
    a = (m, k) if b == 1 else (b, m, k)
    bb = (k, n) if (b == 1 or plan["b_shared"]) else (b, k, n)
    c = (m, n) if b == 1 else (b, m, n)
    return a, bb, c


def _check_tensor(name, t, shape, dtype, device):
    torch = _torch()
    if not isinstance(t, torch.Tensor):
        raise HipGemmError("%s must be a torch tensor" % name)
    if t.dtype != dtype:
        raise HipGemmError("%s must be %s (got %s)" % (name, dtype, t.dtype))
    if tuple(t.shape) != tuple(shape):
        raise HipGemmError("%s has shape %s, plan needs %s" % (name, tuple(t.shape), tuple(shape)))
    if t.device != device:
        raise HipGemmError("%s is on %s, expected %s" % (name, t.device, device))
    if t.dim() and t.stride(-1) != 1:
        raise HipGemmError("%s must have unit stride in its last dimension" % name)


class PackedB:
    """Weights B packed for the decode kernel (vt_pack_b_i8's layout).

    `data` is a flat int8 device tensor of `batch` packed matrices of
    `size_bytes` each: for every 16-column block and 64-row block of the K x N
    matrix, one 1 KiB tile holding the v_mfma_i32_16x16x64_i8 B operand
    (include/vt_hip_gemm.h gives the byte formula). Build it with pack_b.
    """

    __slots__ = ("data", "k", "n", "batch")

    def __init__(self, data, k, n, batch=1):
        self.data, self.k, self.n, self.batch = data, k, n, batch

    @property
    def size_bytes(self):
        """Bytes of one packed matrix: n * (k rounded up to 64)."""
        return self.n * (-(-self.k // 64) * 64)

    @property
    def device(self):
        return self.data.device

    def __repr__(self):
        return "PackedB(k=%d, n=%d, batch=%d, device=%s)" % (self.k, self.n, self.batch,
                                                            self.data.device)


def pack_b(B, *, out=None, stream=None):
    """Pack row-major int8 B [k, n] (or [batch, k, n]) for the skinny_packed variant.

    Runs vt_pack_b_i8 on B's GPU; raises HipGemmError for host tensors or
    shapes the format refuses (n must be a multiple of 16). The packed copy
    is computed once and reused by every call with these weights. `out`, a
    PackedB of the same shape, is repacked in place instead of allocating.
    """
    torch = _torch()
    if not isinstance(B, torch.Tensor) or B.dtype != torch.int8 or B.dim() not in (2, 3):
        raise HipGemmError("B must be an int8 torch tensor [k, n] or [batch, k, n]")
    if B.device.type != "cuda":
        raise HipGemmError("B must be on a gfx950 GPU (got %s); hip_gemm has no CPU path"
                           % B.device)
    if B.stride(-1) != 1:
        raise HipGemmError("B must have unit stride in its last dimension")
    batch = B.shape[0] if B.dim() == 3 else 1
    k, n = B.shape[-2], B.shape[-1]
    size = _lib.packed_b_size(k, n)
    if out is None:
        data = torch.empty(batch * size, dtype=torch.int8, device=B.device)
    else:
        if not isinstance(out, PackedB) or (out.k, out.n, out.batch) != (k, n, batch):
            raise HipGemmError("out must be a PackedB with k=%d n=%d batch=%d" % (k, n, batch))
        data = out.data
        if (not isinstance(data, torch.Tensor) or data.dtype != torch.int8 or data.dim() != 1
                or data.numel() != batch * size or not data.is_contiguous()
                or data.device != B.device):
            raise HipGemmError("out.data must be a contiguous int8 tensor of %d bytes on %s"
                               % (batch * size, B.device))
    if stream is None:
        with torch.cuda.device(B.device):
            stream = torch.cuda.current_stream(B.device).cuda_stream
    elif out is None:
        _keep_for_stream(data, stream)
    _lib.pack_b_raw(B.data_ptr(), data.data_ptr(), k, n, B.stride(-2), batch,
                    B.stride(0) if B.dim() == 3 else 0, size, stream)
    return out if out is not None else PackedB(data, k, n, batch)


def _keep_for_stream(t, stream):
    """t was allocated on torch's current stream but is written on the
    caller's raw stream: record that use, so the caching allocator does not
    hand t's memory out again while that stream may still be writing it."""
    torch = _torch()
    with torch.cuda.device(t.device):
        if stream != torch.cuda.current_stream(t.device).cuda_stream:
            t.record_stream(torch.cuda.ExternalStream(stream, device=t.device))


def _check_packed(B, plan, device):
    torch = _torch()
    if not isinstance(B, PackedB):
        raise HipGemmError("variant %r needs B packed by pack_b (got %s)"
                           % (PACKED_VARIANT, type(B).__name__))
    want_batch = 1 if (plan["batch"] == 1 or plan["b_shared"]) else plan["batch"]
    if (B.k, B.n, B.batch) != (plan["k"], plan["n"], want_batch):
        raise HipGemmError("packed B is k=%d n=%d batch=%d, plan needs k=%d n=%d batch=%d"
                           % (B.k, B.n, B.batch, plan["k"], plan["n"], want_batch))
    data = B.data
    if (not isinstance(data, torch.Tensor) or data.dtype != torch.int8 or data.dim() != 1
            or data.numel() != B.batch * B.size_bytes or not data.is_contiguous()):
        raise HipGemmError("packed B data must be a contiguous int8 tensor of %d bytes"
                           % (B.batch * B.size_bytes))
    if data.device != device:
        raise HipGemmError("packed B is on %s, expected %s" % (data.device, device))


def native_runner(plan, A, B, D, C, stream):
    """Default device runner: one vt_gemm_i8 (or vt_gemm_i8_packed) call
    through the C ABI."""
    m, n, k, b = plan["m"], plan["n"], plan["k"], plan["batch"]
    if plan["variant"] == PACKED_VARIANT:
        ldd = D.stride(-2) if D is not None else n
        sbp = B.size_bytes if B.batch > 1 else 0
        _lib.gemm_packed_raw(A.data_ptr(), B.data.data_ptr(),
                             D.data_ptr() if D is not None else None, C.data_ptr(),
                             m, n, k, A.stride(-2), ldd, C.stride(-2), b,
                             A.stride(0) if b > 1 else 0, sbp,
                             D.stride(0) if (D is not None and b > 1) else 0,
                             C.stride(0) if b > 1 else 0, plan["k_split"], stream)
        return
    lda = A.stride(-2)
    ldb = B.stride(-2)
    ldc = C.stride(-2)
    ldd = D.stride(-2) if D is not None else n
    sa = A.stride(0) if b > 1 else 0
    sb = B.stride(0) if (b > 1 and B.dim() == 3) else 0
    sc = C.stride(0) if b > 1 else 0
    sd = D.stride(0) if (D is not None and b > 1) else 0
    _lib.gemm_raw(A.data_ptr(), B.data_ptr(), D.data_ptr() if D is not None else None,
                  C.data_ptr(), m, n, k, lda, ldb, ldd, ldc, b, sa, sb, sd, sc,
                  plan["variant"], plan["k_split"], stream)


def run(plan, A, B, D=None, *, out=None, stream=None, runner=None):
    """C = D + A.B on the GPU for device tensors; returns C (int32).

    Fails closed like run_commands (backend.py:433-445): the plan is
    validated first and any mismatch raises HipGemmError before a kernel is
    launched. `runner` (plan, A, B, D, C, stream) replaces the native call
    (dependency injection for host-only tests); `stream` is a raw hipStream_t
    handle, default torch's current stream. On another stream the caller
    orders the operands' producers before it, as with any raw stream; a C
    allocated here is recorded as used on that stream.
    """
    ok, reason = validate_plan(plan)
    if not ok:
        raise HipGemmError("invalid plan: " + reason)
    torch = _torch()
    if not isinstance(A, torch.Tensor):
        raise HipGemmError("A must be a torch tensor")
    device = A.device
    a_shape, b_shape, c_shape = _operand_shapes(plan)
    _check_tensor("A", A, a_shape, torch.int8, device)
    if plan["variant"] == PACKED_VARIANT:
        _check_packed(B, plan, device)
    else:
        if isinstance(B, PackedB):
            raise HipGemmError("a packed B needs variant %r (plan has %r)"
                               % (PACKED_VARIANT, plan["variant"]))
        _check_tensor("B", B, b_shape, torch.int8, device)
    if plan["has_d"]:
        if D is None:
            raise HipGemmError("plan has_d=True but D is None")
        _check_tensor("D", D, c_shape, torch.int32, device)
    elif D is not None:
        raise HipGemmError("plan has_d=False but D was given")
    allocated = out is None
    if allocated:
        out = torch.empty(c_shape, dtype=torch.int32, device=device)
    else:
        _check_tensor("out", out, c_shape, torch.int32, device)
    if runner is None:
        if device.type != "cuda":
            raise HipGemmError("operands must be on a gfx950 GPU (got %s); hip_gemm has "
                               "no CPU path" % device)
        runner = native_runner
        if stream is None:
            with torch.cuda.device(device):
                stream = torch.cuda.current_stream(device).cuda_stream
        elif allocated:
            _keep_for_stream(out, stream)
    runner(plan, A, B, D, out, stream)
    return out


def run_flat(plan, A, B, D=None):
    """Flat-list form of run (the reference's ownership convention,
    backend.py:394 / :562): int lists in, a fresh int list out."""
    torch = _torch()
    import numpy as np
    a_shape, b_shape, c_shape = _operand_shapes(plan)
    for name, vals, n in (("A", A, math.prod(a_shape)), ("B", B, math.prod(b_shape))):
        if len(vals) != n:
            raise HipGemmError("%s has %d values, plan needs %d" % (name, len(vals), n))
        for v in vals:
            if not _is_int(v) or not ELEM_MIN <= v <= ELEM_MAX:
                raise HipGemmError("int8 input out of [-128,127]: %r" % (v,))
    dev = torch.device("cuda", torch.cuda.current_device()) if torch.cuda.is_available() else None
    if dev is None:
        raise HipGemmError("no GPU available: hip_gemm has no CPU path")
    At = torch.from_numpy(np.asarray(A, dtype=np.int8).reshape(a_shape)).to(dev)
    Bt = torch.from_numpy(np.asarray(B, dtype=np.int8).reshape(b_shape)).to(dev)
    Dt = None
    if D is not None:
        Dt = torch.from_numpy(np.asarray(D, dtype=np.int32).reshape(c_shape)).to(dev)
    C = run(plan, At, Bt, Dt)
    torch.cuda.synchronize(dev)
    return C.cpu().reshape(-1).tolist()
