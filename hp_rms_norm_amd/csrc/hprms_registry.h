// hprms_registry.h - the instantiated vector-tier kernels of the fused
// add + RMSNorm family: (dtype, mode, shape, flags) -> kernel.  Shared by
// hprms.hip (the 128-byte-aligned kernels and the dispatch),
// hprms_unaligned.hip and hprms_tail.hip (the variants for every other row
// layout), which the build compiles in parallel.
#pragma once

#include "hprms_kernels.h"

namespace hprms {

typedef void (*fused_fn)(const uint16_t*, uint16_t*, const uint16_t*, int64_t, int32_t, int32_t, int32_t, int32_t,
                         uint32_t, float, FusedArgs);

struct FusedEntry {
  int dtype, mode, lpr, vpl, ldsv, block, flags;
  fused_fn fn;
};

// flags: bits 0-1 = non-temporal loads / stores, bit 2 = weight loaded late,
// bits 3-4 = sc1 policy bit on the row loads / stores, bit 5 = the variant for
// rows that are not 128-byte aligned (any 2-byte boundary), bit 6 = with the
// tail vector for hidden % 8 != 0 (with bit 5), bit 7 = residual loads first,
// bit 8 = held to 8 waves per SIMD, bit 9 = timeline instrumentation (bench
// library only), bit 10 = row groups in the xor XCD order (bench library),
// bit 11 = one workgroup per CU (the launch reserves LDS),
// bit 12 = the output phase's separate unpack (bench library), bit 13 = sc0 on
// the stores (bench library), bit 14 = the tail variant's weight staged in
// LDS, bit 15 = the partial sums' parts loaded before any is added, bits
// 16-18 = V > 0: row groups in runs of 2^V per XCD (xcd_runs; the product
// has two, hprms.hip kRuns),
// bit 19 = the output phase at raised wave priority (bench library), bits 20
// / 21 = the two load orders alternating per wave / per workgroup (with bit 7;
// bench library)
#define HPRMS_FUSED_ENTRY(DT, MODE, LPR, VPL, LDSV, BLOCK, FLAGS)                             \
  {DT, MODE, LPR, VPL, LDSV, BLOCK, FLAGS,                                                   \
   &fused_vec_kernel<DT, MODE, LPR, VPL, LDSV, BLOCK, (FLAGS) & ~4, ((FLAGS) >> 2) & 1>},

// The unaligned variants of a shape: the same lanes, vectors and weight
// timing, bit 5 set (which also rotates each row's lane mapping onto 512-byte
// boundaries in modes 0, 1, 3 and 4); and the same with the tail (bit 6),
// which costs about 30 VGPRs and so is kept apart from the rows that need no
// tail.  Every shape has them without the sc1 bits (the FP8 and MX variants,
// which write partial cache lines, and calls small enough to stay in the
// Infinity Cache); the rotated modes' shapes with sc1 also have them with it.
#define HPRMS_UNALIGNED_ENTRY(DT, MODE, LPR, VPL, LDSV, BLOCK, FLAGS) \
  HPRMS_FUSED_ENTRY(DT, MODE, LPR, VPL, LDSV, BLOCK, ((FLAGS) & ~24) | 32)
#define HPRMS_TAIL_ENTRY(DT, MODE, LPR, VPL, LDSV, BLOCK, FLAGS) \
  HPRMS_FUSED_ENTRY(DT, MODE, LPR, VPL, LDSV, BLOCK, ((FLAGS) & ~24) | 96)
#define HPRMS_UNALIGNED_SC1_ENTRY(DT, MODE, LPR, VPL, LDSV, BLOCK, FLAGS) \
  HPRMS_FUSED_ENTRY(DT, MODE, LPR, VPL, LDSV, BLOCK, (FLAGS) | 32)
#define HPRMS_TAIL_SC1_ENTRY(DT, MODE, LPR, VPL, LDSV, BLOCK, FLAGS) \
  HPRMS_FUSED_ENTRY(DT, MODE, LPR, VPL, LDSV, BLOCK, (FLAGS) | 96)
// tail variants with the weight staged in LDS (flags bit 14)
#define HPRMS_TAIL_WLDS_ENTRY(DT, MODE, LPR, VPL, LDSV, BLOCK, FLAGS) \
  HPRMS_FUSED_ENTRY(DT, MODE, LPR, VPL, LDSV, BLOCK, ((FLAGS) & ~24) | 96 | 16384)
#define HPRMS_TAIL_WLDS_SC1_ENTRY(DT, MODE, LPR, VPL, LDSV, BLOCK, FLAGS) \
  HPRMS_FUSED_ENTRY(DT, MODE, LPR, VPL, LDSV, BLOCK, (FLAGS) | 96 | 16384)

// (lanes per row, vectors per lane, of which in LDS, block, flags).  flags 3 =
// nt on the row loads and stores, 7 = the same with the weight loaded late,
// 27 / 31 = nt plus sc1 on loads and stores (without / with the late weight);
// +128 = the residual's loads issued before the input's.
//
// Per mode, exactly the shapes its dispatch table (hprms.hip) can choose:
// the rows every mode shares, then each mode's own.  A CPU test enumerates the
// tables and checks that these lists hold every reachable shape and no other.
#define HPRMS_COMMON_BW_SHAPES(X, DT, MODE)                                                      \
  X(DT, MODE, 16, 1, 0, 256, 3) X(DT, MODE, 32, 1, 0, 256, 3) X(DT, MODE, 64, 1, 0, 256, 3)      \
  X(DT, MODE, 32, 4, 0, 256, 131) X(DT, MODE, 512, 3, 0, 512, 159) X(DT, MODE, 1024, 8, 4, 1024, 31)
// the latency rows (hprms.hip, latency_config; FL = 32768 for the partial sums,
// which load all parts before adding them)
#define HPRMS_LATENCY_SHAPES(X, DT, MODE, FL)                                                     \
  X(DT, MODE, 64, 2, 0, 64, 3 | FL) X(DT, MODE, 128, 2, 0, 128, 3 | FL) X(DT, MODE, 256, 2, 0, 256, 7 | FL) \
  X(DT, MODE, 512, 2, 0, 512, 7 | FL) X(DT, MODE, 512, 4, 0, 512, 7 | FL)
#define HPRMS_COMMON_SHAPES(X, DT, MODE) HPRMS_COMMON_BW_SHAPES(X, DT, MODE) HPRMS_LATENCY_SHAPES(X, DT, MODE, 0)

// the fused op in place (mode 0) and its out-of-place (3) and partial-sum (4)
// forms.  In 1024 x 2 and 1024 x 3 these modes load the weight with the row
// (flags 27 / 155) except in the tail variants (31 / 159), which have no
// LDS-tier 256 x 8 either (hprms.hip, table_config and tail_shape).
#define HPRMS_FUSED_ROWS(X, DT, MODE, F2, F3, FL)                                                 \
  HPRMS_COMMON_BW_SHAPES(X, DT, MODE) HPRMS_LATENCY_SHAPES(X, DT, MODE, FL)                        \
  X(DT, MODE, 64, 4, 0, 256, 135) X(DT, MODE, 128, 3, 0, 256, 7) X(DT, MODE, 1024, 2, 0, 1024, F2) \
  X(DT, MODE, 1024, 3, 0, 1024, F3) X(DT, MODE, 1024, 4, 0, 1024, 159)
#define HPRMS_FUSED_TAIL_SHAPES(X, DT, MODE) HPRMS_FUSED_ROWS(X, DT, MODE, 31, 159, 0)
#define HPRMS_MODE4_TAIL_SHAPES(X, DT, MODE) HPRMS_FUSED_ROWS(X, DT, MODE, 31, 159, 32768)
#define HPRMS_FUSED_SHAPES(X, DT, MODE) HPRMS_FUSED_ROWS(X, DT, MODE, 27, 155, 0) X(DT, MODE, 256, 8, 4, 256, 27)
// 32 lanes x 5-12 vectors, two rows per one-wave workgroup: the fused op in
// and out of place at 1K-3K and 1024 < rows <= 4096 (hprms.hip, wide_rows)
#define HPRMS_WIDE_ROWS(X, DT, MODE)                                                              \
  X(DT, MODE, 32, 5, 0, 64, 135) X(DT, MODE, 32, 6, 0, 64, 135) X(DT, MODE, 32, 7, 0, 64, 135)     \
  X(DT, MODE, 32, 8, 0, 64, 135) X(DT, MODE, 32, 9, 0, 64, 135) X(DT, MODE, 32, 10, 0, 64, 135)    \
  X(DT, MODE, 32, 11, 0, 64, 135) X(DT, MODE, 32, 12, 0, 64, 135)
// 64 lanes x 7-10 vectors, one row per one-wave workgroup: the fused op in
// and out of place and plain RMSNorm at 3K-5K and 768 < rows <= 2048 on the
// 128-byte grid
// (hprms.hip, wave_rows; aligned registry only)
#define HPRMS_WAVE_ROWS(X, DT, MODE) \
  X(DT, MODE, 64, 7, 0, 64, 135) X(DT, MODE, 64, 8, 0, 64, 135) X(DT, MODE, 64, 9, 0, 64, 135) \
  X(DT, MODE, 64, 10, 0, 64, 135)
// 128 lanes x 6-8 vectors, one row per two-wave workgroup: the fused op in
// and out of place at 5K-8K and 512 < rows <= 1280 on the 128-byte grid
// (hprms.hip, pair_rows; aligned registry only)
#define HPRMS_PAIR_ROWS(X, DT, MODE) \
  X(DT, MODE, 128, 6, 0, 128, 135) X(DT, MODE, 128, 7, 0, 128, 135) X(DT, MODE, 128, 8, 0, 128, 135)
// the in-place op's rows with their row groups in runs per XCD (hprms.hip, kRuns)
#define HPRMS_RUNS_ROWS(X, DT, MODE) X(DT, MODE, 256, 2, 0, 256, 131 | 327680) X(DT, MODE, 512, 2, 0, 512, 7 | 393216)
// the quantised outputs' rows with runs of 32 row groups per XCD (hprms.hip,
// kRuns; aligned registry only): 16 KiB rows in modes 2, 5, 6, 7, and 8 KiB
// rows in mode 7 (column-major scales)
#define HPRMS_QUANT_RUNS(X, DT)                                                                    \
  X(DT, 2, 512, 2, 0, 512, 7 | 327680) X(DT, 5, 512, 2, 0, 512, 7 | 327680)                       \
  X(DT, 6, 512, 2, 0, 512, 7 | 327680) X(DT, 7, 512, 2, 0, 512, 7 | 327680)                       \
  X(DT, 7, 256, 2, 0, 256, 7 | 327680)
// bench library: the same runs where the table leaves them out (modes 2, 5, 6
// at 8 KiB rows; mode 7 at 32 and 64 KiB rows), and runs of 32 and 64 for the
// plain RMSNorm (mode 1) and the op out of place (mode 3) at 8 and 16 KiB
// rows, for bench.py --ab-runs
#define HPRMS_QUANT_RUNS_AB(X, DT)                                                                 \
  X(DT, 2, 256, 2, 0, 256, 7 | 327680) X(DT, 5, 256, 2, 0, 256, 7 | 327680)                       \
  X(DT, 6, 256, 2, 0, 256, 7 | 327680) X(DT, 7, 1024, 2, 0, 1024, 31 | 327680)                    \
  X(DT, 7, 1024, 4, 0, 1024, 159 | 327680)                                                        \
  X(DT, 1, 64, 8, 0, 256, 3 | 327680) X(DT, 1, 64, 8, 0, 256, 3 | 393216)                         \
  X(DT, 1, 512, 2, 0, 512, 31 | 327680) X(DT, 1, 512, 2, 0, 512, 31 | 393216)                     \
  X(DT, 3, 128, 4, 0, 256, 131 | 327680) X(DT, 3, 128, 4, 0, 256, 131 | 393216)                   \
  X(DT, 3, 512, 2, 0, 512, 7 | 327680) X(DT, 3, 512, 2, 0, 512, 7 | 393216)
#define HPRMS_MODE0_SHAPES(X, DT, MODE) HPRMS_FUSED_SHAPES(X, DT, MODE) X(DT, MODE, 256, 2, 0, 256, 131) \
  HPRMS_WIDE_ROWS(X, DT, MODE) HPRMS_WAVE_ROWS(X, DT, MODE) HPRMS_PAIR_ROWS(X, DT, MODE) HPRMS_RUNS_ROWS(X, DT, MODE)
// rows off the 128-byte grid at 3K < H <= 4K keep 128 x 4 in place (hprms.hip, inplace_config)
#define HPRMS_MODE0_OFFGRID_SHAPES(X, DT, MODE) \
  HPRMS_FUSED_SHAPES(X, DT, MODE) X(DT, MODE, 128, 4, 0, 256, 131) HPRMS_WIDE_ROWS(X, DT, MODE)
#define HPRMS_MODE3_SHAPES(X, DT, MODE) \
  HPRMS_FUSED_SHAPES(X, DT, MODE) X(DT, MODE, 128, 4, 0, 256, 131) HPRMS_WIDE_ROWS(X, DT, MODE)
#define HPRMS_MODE4_SHAPES(X, DT, MODE)                                                           \
  HPRMS_FUSED_ROWS(X, DT, MODE, 27, 155, 32768) X(DT, MODE, 256, 8, 4, 256, 27)                   \
  X(DT, MODE, 128, 4, 0, 256, 131) X(DT, MODE, 256, 4, 0, 256, 3)

// plain RMSNorm (mode 1)
#define HPRMS_MODE1_SHAPES(X, DT, MODE)                                                           \
  HPRMS_COMMON_SHAPES(X, DT, MODE) X(DT, MODE, 1024, 3, 0, 1024, 159)                              \
  X(DT, MODE, 64, 4, 0, 256, 135) X(DT, MODE, 64, 8, 0, 256, 3) X(DT, MODE, 256, 3, 0, 256, 7)      \
  X(DT, MODE, 512, 2, 0, 512, 31) X(DT, MODE, 512, 4, 0, 512, 31) X(DT, MODE, 512, 8, 0, 512, 7)

// the FP8 output (mode 2) and the OCP MX outputs (modes 5 and 6)
#define HPRMS_QUANT_SHAPES(X, DT, MODE)                                                           \
  HPRMS_COMMON_SHAPES(X, DT, MODE) X(DT, MODE, 1024, 3, 0, 1024, 159)                              \
  X(DT, MODE, 128, 3, 0, 256, 7) X(DT, MODE, 256, 3, 0, 256, 7) X(DT, MODE, 1024, 2, 0, 1024, 31)
#define HPRMS_MODE2_SHAPES(X, DT, MODE) HPRMS_QUANT_SHAPES(X, DT, MODE) X(DT, MODE, 512, 8, 4, 512, 159)
#define HPRMS_MX_SHAPES(X, DT, MODE) HPRMS_QUANT_SHAPES(X, DT, MODE) X(DT, MODE, 1024, 4, 0, 1024, 159)

// Every mode's lists for one registry: the kernels for rows on the 128-byte
// grid (ENTRY = HPRMS_FUSED_ENTRY), and for rows off it (the unaligned and
// tail entries below; the tail variant has no MX form).
#define HPRMS_MODES_1_TO_4(ENTRY, DT)                                                             \
  HPRMS_MODE1_SHAPES(ENTRY, DT, 1) HPRMS_MODE2_SHAPES(ENTRY, DT, 2) HPRMS_MODE3_SHAPES(ENTRY, DT, 3) \
  HPRMS_MODE4_SHAPES(ENTRY, DT, 4)
#define HPRMS_ALL_MODES(ENTRY, DT) \
  HPRMS_MODE0_SHAPES(ENTRY, DT, 0) HPRMS_MODES_1_TO_4(ENTRY, DT) HPRMS_WAVE_ROWS(ENTRY, DT, 3) \
  HPRMS_WAVE_ROWS(ENTRY, DT, 1) \
  HPRMS_PAIR_ROWS(ENTRY, DT, 3)
#define HPRMS_ALL_MODES_OFFGRID(ENTRY, DT) HPRMS_MODE0_OFFGRID_SHAPES(ENTRY, DT, 0) HPRMS_MODES_1_TO_4(ENTRY, DT)
#define HPRMS_ALL_MODES_TAIL(ENTRY, DT)                                                           \
  HPRMS_FUSED_TAIL_SHAPES(ENTRY, DT, 0) ENTRY(DT, 0, 128, 4, 0, 256, 131) HPRMS_WIDE_ROWS(ENTRY, DT, 0) \
  HPRMS_MODE1_SHAPES(ENTRY, DT, 1) HPRMS_MODE2_SHAPES(ENTRY, DT, 2)                              \
  HPRMS_FUSED_TAIL_SHAPES(ENTRY, DT, 3) ENTRY(DT, 3, 128, 4, 0, 256, 131) HPRMS_WIDE_ROWS(ENTRY, DT, 3) \
  HPRMS_MODE4_TAIL_SHAPES(ENTRY, DT, 4) ENTRY(DT, 4, 128, 4, 0, 256, 131) ENTRY(DT, 4, 256, 4, 0, 256, 3)
// the block-scaled outputs: MX (modes 5, 6) and FP8 with a scale per 128
// elements (mode 7), with the same shapes
#define HPRMS_MX_MODES(ENTRY, DT) \
  HPRMS_MX_SHAPES(ENTRY, DT, 5) HPRMS_MX_SHAPES(ENTRY, DT, 6) HPRMS_MX_SHAPES(ENTRY, DT, 7)

// The shapes with sc1 bits among the lists of modes 0, 1, 3 and 4 (their
// off-grid variants keep them for calls past the Infinity Cache)
#define HPRMS_SC1_COMMON_SHAPES(X, DT, MODE) X(DT, MODE, 512, 3, 0, 512, 159) X(DT, MODE, 1024, 8, 4, 1024, 31)
#define HPRMS_SC1_FUSED_SHAPES(X, DT, MODE)                                                       \
  HPRMS_SC1_COMMON_SHAPES(X, DT, MODE) X(DT, MODE, 1024, 3, 0, 1024, 155)                         \
  X(DT, MODE, 1024, 2, 0, 1024, 27) X(DT, MODE, 256, 8, 4, 256, 27) X(DT, MODE, 1024, 4, 0, 1024, 159)
#define HPRMS_SC1_MODE1_SHAPES(X, DT, MODE)                                                       \
  HPRMS_SC1_COMMON_SHAPES(X, DT, MODE) X(DT, MODE, 1024, 3, 0, 1024, 159)                         \
  X(DT, MODE, 512, 2, 0, 512, 31) X(DT, MODE, 512, 4, 0, 512, 31)
#define HPRMS_ROTATED_MODES_SC1(ENTRY, DT)                                                         \
  HPRMS_SC1_FUSED_SHAPES(ENTRY, DT, 0) HPRMS_SC1_MODE1_SHAPES(ENTRY, DT, 1)                      \
  HPRMS_SC1_FUSED_SHAPES(ENTRY, DT, 3) HPRMS_SC1_FUSED_SHAPES(ENTRY, DT, 4)
// the same for the tail variants, which keep sc1 only past 2048 whole vectors
// (plain RMSNorm's 1024 x 3 tail then stages its weight in LDS: HPRMS_WLDS_TAIL_SC1)
#define HPRMS_SC1_TAIL_FUSED_SHAPES(X, DT, MODE)                                                  \
  X(DT, MODE, 1024, 3, 0, 1024, 159) X(DT, MODE, 1024, 8, 4, 1024, 31) X(DT, MODE, 1024, 4, 0, 1024, 159)
#define HPRMS_ROTATED_MODES_SC1_TAIL(ENTRY, DT)                                                    \
  HPRMS_SC1_TAIL_FUSED_SHAPES(ENTRY, DT, 0) ENTRY(DT, 1, 1024, 8, 4, 1024, 31)                   \
  HPRMS_SC1_TAIL_FUSED_SHAPES(ENTRY, DT, 3) HPRMS_SC1_TAIL_FUSED_SHAPES(ENTRY, DT, 4)

// The tail shapes that stage the weight in LDS from 1024 rows (plain RMSNorm:
// 384; hprms.hip, tail_shape): 512 x 2, 512 x 3 and 1024 x 2 in the fused op
// in place and out of place, 512 x 3 in the partial-sum form, and 512 x 2, 3
// and 4 and 1024 x 3 in plain RMSNorm (its 1024 x 3 also with sc1).
#define HPRMS_WLDS_FUSED_SHAPES(X, DT, MODE) \
  X(DT, MODE, 512, 2, 0, 512, 7) X(DT, MODE, 512, 3, 0, 512, 159) X(DT, MODE, 1024, 2, 0, 1024, 31)
#define HPRMS_ALL_MODES_WLDS_TAIL(ENTRY, DT)                                                      \
  HPRMS_WLDS_FUSED_SHAPES(ENTRY, DT, 0) HPRMS_WLDS_FUSED_SHAPES(ENTRY, DT, 3)                    \
  ENTRY(DT, 4, 512, 3, 0, 512, 159)                                                              \
  ENTRY(DT, 1, 512, 2, 0, 512, 31) ENTRY(DT, 1, 512, 3, 0, 512, 159) ENTRY(DT, 1, 512, 4, 0, 512, 31) \
  ENTRY(DT, 1, 1024, 3, 0, 1024, 159)
#define HPRMS_WLDS_TAIL_SC1(ENTRY, DT) ENTRY(DT, 1, 1024, 3, 0, 1024, 159)

// Bench library: the shapes the other modes choose, as in-place (mode 0)
// kernels, so a test can run the 16-bit op with another form's lane mapping
// (and so the same fp32 reduction order) as that form's bit-level reference.
#define HPRMS_OTHER_MODE_SHAPES(X, DT, MODE)                                                      \
  X(DT, MODE, 128, 4, 0, 256, 131) X(DT, MODE, 256, 4, 0, 256, 3) X(DT, MODE, 256, 3, 0, 256, 7)  \
  X(DT, MODE, 512, 8, 4, 512, 159) X(DT, MODE, 64, 8, 0, 256, 3) X(DT, MODE, 512, 2, 0, 512, 31)  \
  X(DT, MODE, 512, 4, 0, 512, 31) X(DT, MODE, 512, 8, 0, 512, 7) X(DT, MODE, 1024, 2, 0, 1024, 31) \
  X(DT, MODE, 1024, 3, 0, 1024, 159)

// The shapes below are built only into the bench library libhprms_bench.so
// (hprms.hip compiled with HPRMS_BENCH_BUILD), never into libhprms.so: no
// table row selects them.
//
// Alternatives of the fused op that the tuning sweeps compare against (five
// of the table's shapes with the two streams' loads alternating, the two
// smallest latency rows with the weight loaded late, and other lane shapes).
#define HPRMS_ALT_SHAPES(X, DT, MODE)                                                          \
  X(DT, MODE, 64, 2, 0, 256, 3) X(DT, MODE, 256, 8, 0, 256, 27)                               \
  X(DT, MODE, 512, 8, 4, 512, 31) X(DT, MODE, 1024, 8, 0, 1024, 31)                           \
  X(DT, MODE, 32, 4, 0, 256, 3) X(DT, MODE, 64, 4, 0, 256, 7) X(DT, MODE, 128, 4, 0, 256, 3)   \
  X(DT, MODE, 1024, 3, 0, 1024, 31) X(DT, MODE, 1024, 4, 0, 1024, 31)                         \
  X(DT, MODE, 64, 2, 0, 64, 7) X(DT, MODE, 128, 2, 0, 128, 7) X(DT, MODE, 512, 8, 4, 512, 159)

// other cache policies and LDS splits of the fused op (bf16)
#define HPRMS_TUNING_SHAPES(X, DT, MODE)                                                        \
  X(DT, MODE, 64, 2, 0, 256, 11) X(DT, MODE, 128, 4, 0, 256, 27) X(DT, MODE, 256, 4, 0, 256, 27) \
  X(DT, MODE, 512, 4, 0, 512, 3) X(DT, MODE, 1024, 4, 0, 1024, 7) X(DT, MODE, 512, 4, 0, 512, 27) \
  X(DT, MODE, 256, 16, 8, 256, 31) X(DT, MODE, 128, 4, 0, 256, 0) X(DT, MODE, 1024, 4, 2, 1024, 31) \
  X(DT, MODE, 256, 6, 3, 256, 31) X(DT, MODE, 256, 8, 4, 256, 3)

// candidates of the table's rows (bf16): +256 = held to 8 waves per SIMD,
// +2048 = one workgroup per CU (the launch reserves 96 KiB of LDS), other
// cache policies of the 3K-12K rows (sc1 on the stores alone: +16; sc0 on the
// stores: +8192; no nt on the loads, the stores or either), and the latency
// rows of 4K-8K with the weight loaded with the row (flags 3)
#define HPRMS_CANDIDATE_SHAPES(X, DT, MODE)                                                          \
  X(DT, MODE, 32, 4, 0, 256, 135) X(DT, MODE, 64, 4, 0, 256, 131) X(DT, MODE, 128, 2, 0, 256, 135)    \
  X(DT, MODE, 128, 4, 0, 256, 135) X(DT, MODE, 128, 4, 0, 256, 159) X(DT, MODE, 128, 4, 0, 256, 391) \
  X(DT, MODE, 256, 2, 0, 256, 131) X(DT, MODE, 256, 2, 0, 256, 135) X(DT, MODE, 256, 2, 0, 256, 155)  \
  X(DT, MODE, 256, 2, 0, 256, 159) X(DT, MODE, 256, 4, 0, 256, 135) X(DT, MODE, 256, 4, 0, 256, 159)  \
  X(DT, MODE, 512, 2, 0, 512, 135) X(DT, MODE, 512, 2, 0, 512, 159) X(DT, MODE, 256, 6, 0, 256, 159)  \
  X(DT, MODE, 512, 3, 0, 512, 159) X(DT, MODE, 512, 4, 0, 512, 159) X(DT, MODE, 1024, 2, 0, 1024, 159) \
  X(DT, MODE, 1024, 2, 0, 1024, 2079) X(DT, MODE, 1024, 3, 0, 1024, 2207) X(DT, MODE, 1024, 4, 0, 1024, 2207) \
  X(DT, MODE, 256, 8, 4, 256, 155) X(DT, MODE, 256, 12, 0, 256, 159) X(DT, MODE, 512, 6, 0, 512, 159)         \
  X(DT, MODE, 128, 3, 0, 256, 23) X(DT, MODE, 128, 3, 0, 256, 31) X(DT, MODE, 256, 2, 0, 256, 147)            \
  X(DT, MODE, 512, 2, 0, 512, 23) X(DT, MODE, 512, 3, 0, 512, 143) X(DT, MODE, 512, 3, 0, 512, 135)           \
  X(DT, MODE, 256, 2, 0, 256, 8323) X(DT, MODE, 512, 2, 0, 512, 8199) X(DT, MODE, 128, 3, 0, 256, 8199)        \
  X(DT, MODE, 256, 2, 0, 256, 8339) X(DT, MODE, 512, 2, 0, 512, 8215)                                        \
  X(DT, MODE, 256, 2, 0, 256, 128) X(DT, MODE, 256, 2, 0, 256, 129) X(DT, MODE, 256, 2, 0, 256, 130)           \
  X(DT, MODE, 32, 4, 0, 256, 128) X(DT, MODE, 32, 4, 0, 256, 129) X(DT, MODE, 32, 4, 0, 256, 130)              \
  X(DT, MODE, 512, 2, 0, 512, 4) X(DT, MODE, 512, 2, 0, 512, 5) X(DT, MODE, 512, 2, 0, 512, 6)          \
  X(DT, MODE, 256, 2, 0, 256, 3) X(DT, MODE, 512, 2, 0, 512, 3)

// the bandwidth table's rows with the output phase's separate unpack (+4096)
#define HPRMS_SHARED_UNPACK_SHAPES(X, DT, MODE)                                                        \
  X(DT, MODE, 32, 4, 0, 256, 4227) X(DT, MODE, 64, 4, 0, 256, 4231) X(DT, MODE, 128, 3, 0, 256, 4103)   \
  X(DT, MODE, 128, 4, 0, 256, 4227) X(DT, MODE, 512, 2, 0, 512, 4103) X(DT, MODE, 512, 3, 0, 512, 4127) \
  X(DT, MODE, 1024, 2, 0, 1024, 4127) X(DT, MODE, 256, 8, 4, 256, 4123) X(DT, MODE, 1024, 3, 0, 1024, 4255) \
  X(DT, MODE, 1024, 4, 0, 1024, 4255) X(DT, MODE, 256, 2, 0, 256, 4251) X(DT, MODE, 256, 8, 4, 256, 4251)

// the bandwidth table's rows with the timeline instrumentation (+512)
#define HPRMS_TIMELINE_SHAPES(X, DT, MODE)                                                        \
  X(DT, MODE, 32, 4, 0, 256, 643) X(DT, MODE, 64, 4, 0, 256, 647) X(DT, MODE, 128, 3, 0, 256, 519) \
  X(DT, MODE, 256, 2, 0, 256, 643) X(DT, MODE, 512, 2, 0, 512, 519) X(DT, MODE, 512, 3, 0, 512, 671) \
  X(DT, MODE, 1024, 2, 0, 1024, 539) X(DT, MODE, 256, 8, 4, 256, 539) X(DT, MODE, 1024, 3, 0, 1024, 667) \
  X(DT, MODE, 1024, 4, 0, 1024, 671) X(DT, MODE, 128, 4, 0, 256, 643) X(DT, MODE, 32, 8, 0, 64, 647)   \
  X(DT, MODE, 32, 12, 0, 64, 647)

// every split of a 512-vector row (H = 4096) into lanes x vectors, in
// workgroups of one to eight rows (the grid-size map of the fill-and-drain
// cost at 4096 rows; nt, residual loads first, weight with the row)
#define HPRMS_FILL_SHAPES(X, DT, MODE)                                                            \
  X(DT, MODE, 64, 8, 0, 64, 131) X(DT, MODE, 64, 8, 0, 128, 131) X(DT, MODE, 64, 8, 0, 256, 131)   \
  X(DT, MODE, 64, 8, 0, 512, 131) X(DT, MODE, 128, 4, 0, 128, 131) X(DT, MODE, 128, 4, 0, 256, 131) \
  X(DT, MODE, 128, 4, 0, 512, 131) X(DT, MODE, 256, 2, 0, 512, 131) X(DT, MODE, 512, 1, 0, 512, 131)

// the bandwidth table's rows with their row groups in xcd_xor's order
// (+1024) and in xcd_runs<V>'s (+V << 16: runs of 2^V row groups per XCD)
#define HPRMS_XCD_ORDER_ROWS(X, DT, MODE, F)                                                       \
  X(DT, MODE, 32, 4, 0, 256, 131 | F) X(DT, MODE, 32, 8, 0, 64, 135 | F) X(DT, MODE, 32, 12, 0, 64, 135 | F) \
  X(DT, MODE, 256, 2, 0, 256, 131 | F) X(DT, MODE, 512, 2, 0, 512, 7 | F) X(DT, MODE, 512, 3, 0, 512, 159 | F) \
  X(DT, MODE, 1024, 2, 0, 1024, 27 | F) X(DT, MODE, 256, 8, 4, 256, 27 | F)                              \
  X(DT, MODE, 1024, 3, 0, 1024, 155 | F) X(DT, MODE, 1024, 4, 0, 1024, 159 | F)
#define HPRMS_XCD_ORDER_SHAPES(X, DT, MODE)                                                        \
  HPRMS_XCD_ORDER_ROWS(X, DT, MODE, 1024) HPRMS_XCD_ORDER_ROWS(X, DT, MODE, 65536)                 \
  HPRMS_XCD_ORDER_ROWS(X, DT, MODE, 131072) HPRMS_XCD_ORDER_ROWS(X, DT, MODE, 196608)              \
  HPRMS_XCD_ORDER_ROWS(X, DT, MODE, 262144) HPRMS_XCD_ORDER_ROWS(X, DT, MODE, 327680)              \
  HPRMS_XCD_ORDER_ROWS(X, DT, MODE, 393216) HPRMS_XCD_ORDER_ROWS(X, DT, MODE, 458752)

// candidates at 16384 (LDS splits and weight timing for fewer VGPRs), shapes
// that fit the widths 5K-11K that are not powers of two, and the table's rows
// with the output phase at raised wave priority (+524288)
#define HPRMS_SHAPE_CANDIDATES(X, DT, MODE)                                                        \
  X(DT, MODE, 256, 8, 4, 256, 31) X(DT, MODE, 256, 8, 4, 256, 287) X(DT, MODE, 256, 8, 6, 256, 31)    \
  X(DT, MODE, 256, 8, 6, 256, 27) X(DT, MODE, 512, 4, 2, 512, 31) X(DT, MODE, 512, 4, 2, 512, 27)      \
  X(DT, MODE, 512, 4, 0, 512, 27) X(DT, MODE, 128, 5, 0, 128, 135) X(DT, MODE, 128, 5, 0, 256, 135)    \
  X(DT, MODE, 128, 6, 0, 256, 135) X(DT, MODE, 128, 7, 0, 256, 135) X(DT, MODE, 128, 9, 0, 256, 135)   \
  X(DT, MODE, 256, 5, 0, 256, 135) X(DT, MODE, 128, 10, 0, 256, 135) X(DT, MODE, 256, 3, 0, 256, 135)  \
  X(DT, MODE, 256, 2, 0, 256, 524419) X(DT, MODE, 512, 2, 0, 512, 524295) X(DT, MODE, 512, 3, 0, 512, 524447) \
  X(DT, MODE, 1024, 2, 0, 1024, 524315) X(DT, MODE, 256, 8, 4, 256, 524315)                             \
  X(DT, MODE, 1024, 3, 0, 1024, 524443) X(DT, MODE, 1024, 4, 0, 1024, 524447)
// the bandwidth table's rows with the residual-first and input-first loads
// alternating per wave (+1048576, with +128) and per workgroup (+2097152)
#define HPRMS_ALT_ORDER_ROWS(X, DT, MODE, F)                                                          \
  X(DT, MODE, 256, 2, 0, 256, 131 | F) X(DT, MODE, 512, 2, 0, 512, 135 | F) X(DT, MODE, 512, 3, 0, 512, 159 | F) \
  X(DT, MODE, 1024, 2, 0, 1024, 155 | F) X(DT, MODE, 256, 8, 4, 256, 155 | F)                              \
  X(DT, MODE, 1024, 3, 0, 1024, 155 | F) X(DT, MODE, 1024, 4, 0, 1024, 159 | F)
#define HPRMS_ALT_ORDER_SHAPES(X, DT, MODE) \
  HPRMS_ALT_ORDER_ROWS(X, DT, MODE, 1048576) HPRMS_ALT_ORDER_ROWS(X, DT, MODE, 2097152)

// the latency rows of 4K-8K and the bandwidth rows of 12K-24K with one
// stream's cache policy changed: the input's loads (+4194304) or the
// residual's (+8388608) without nt / sc1, the residual's stores (+16777216)
// or the output's (+33554432) without nt; and the 4K latency row without nt
// on the loads or anywhere
#define HPRMS_STREAM_POLICY_ROWS(X, DT, MODE, F)                                                   \
  X(DT, MODE, 256, 2, 0, 256, 7 | F) X(DT, MODE, 512, 2, 0, 512, 7 | F)                          \
  X(DT, MODE, 512, 3, 0, 512, 159 | F) X(DT, MODE, 1024, 2, 0, 1024, 27 | F)                     \
  X(DT, MODE, 256, 8, 4, 256, 27 | F) X(DT, MODE, 1024, 3, 0, 1024, 155 | F)
#define HPRMS_STREAM_POLICY_SHAPES(X, DT, MODE)                                                   \
  HPRMS_STREAM_POLICY_ROWS(X, DT, MODE, 4194304) HPRMS_STREAM_POLICY_ROWS(X, DT, MODE, 8388608)  \
  HPRMS_STREAM_POLICY_ROWS(X, DT, MODE, 16777216) HPRMS_STREAM_POLICY_ROWS(X, DT, MODE, 33554432) \
  X(DT, MODE, 256, 2, 0, 256, 6) X(DT, MODE, 256, 2, 0, 256, 4)

// The unaligned variants (hprms_unaligned.hip) and the tail variants
// (hprms_tail.hip, modes 0-4: the MX outputs need hidden % 32 == 0): every
// entry the tables can choose, as HPRMS_UNALIGNED_ENTRY / HPRMS_TAIL_ENTRY
// (and the _SC1_ forms) make them.
extern const FusedEntry kFusedUnaligned[];
extern const int kFusedUnalignedCount;
extern const FusedEntry kFusedTail[];
extern const int kFusedTailCount;

}  // namespace hprms
