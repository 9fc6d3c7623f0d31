// hprms.hip - C ABI of libhprms.so: argument checks, the gfx950 dispatch table
// and the kernel launches.  Kernels live in hprms_kernels.h.
//
// Reference interfaces replaced (paths under the reference repository):
//   hprms_fused_add_rmsnorm  <- rms_norm()  hp_rms_norm/csrc/cuda/hp_rms_norm.cu:7-50
//                               launch_rms_norm<T>()  hp_rms_norm/csrc/cuda/hp_rms_norm.cuh:562-618
//   hprms_streamer           <- relu()  hp_rms_norm/csrc/cuda/activation_kernels.cu:7-39
//                               launch_relu<T>()  hp_rms_norm/csrc/cuda/activation_kernels.cuh:122-145
// The other entry points (plain RMSNorm, FP8 output, out of place, partial-sum
// reduction) have no reference counterpart and share the fused kernels.
#include <hip/hip_runtime.h>

#include <atomic>

#include <stdarg.h>
#include <stdlib.h>
#include <stdio.h>
#include <string.h>

#include "hp_rms_norm_amd.h"
#include "hprms_kernels.h"
#include "hprms_registry.h"

namespace hprms {
namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(HPRMS_E_LAUNCH, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  return HPRMS_OK;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
bool aligned2(const void* p) { return ((uintptr_t)p & 1u) == 0; }
// every row starts on a 128-byte boundary (a cache line)
bool rows_aligned128(const void* base, int64_t stride_bytes) {
  return ((uintptr_t)base & 127u) == 0 && stride_bytes % 128 == 0;
}

// Every kernel a dispatch table can choose for rows on the 128-byte grid; the
// bench library (HPRMS_BENCH_BUILD) adds the shapes only the tuning sweeps
// and the ceiling measurements use.
const FusedEntry kFused[] = {
    HPRMS_ALL_MODES(HPRMS_FUSED_ENTRY, HPRMS_DTYPE_BF16)
    HPRMS_ALL_MODES(HPRMS_FUSED_ENTRY, HPRMS_DTYPE_FP16)
    HPRMS_MX_MODES(HPRMS_FUSED_ENTRY, HPRMS_DTYPE_BF16)
    HPRMS_MX_MODES(HPRMS_FUSED_ENTRY, HPRMS_DTYPE_FP16)
    HPRMS_QUANT_RUNS(HPRMS_FUSED_ENTRY, HPRMS_DTYPE_BF16)
    HPRMS_QUANT_RUNS(HPRMS_FUSED_ENTRY, HPRMS_DTYPE_FP16)
#ifdef HPRMS_BENCH_BUILD
    HPRMS_OTHER_MODE_SHAPES(HPRMS_FUSED_ENTRY, HPRMS_DTYPE_BF16, 0)
    HPRMS_OTHER_MODE_SHAPES(HPRMS_FUSED_ENTRY, HPRMS_DTYPE_FP16, 0)
    HPRMS_ALT_SHAPES(HPRMS_FUSED_ENTRY, HPRMS_DTYPE_BF16, 0)
    HPRMS_ALT_SHAPES(HPRMS_FUSED_ENTRY, HPRMS_DTYPE_FP16, 0)
    HPRMS_TUNING_SHAPES(HPRMS_FUSED_ENTRY, HPRMS_DTYPE_BF16, 0)
    HPRMS_CANDIDATE_SHAPES(HPRMS_FUSED_ENTRY, HPRMS_DTYPE_BF16, 0)
    HPRMS_TIMELINE_SHAPES(HPRMS_FUSED_ENTRY, HPRMS_DTYPE_BF16, 0)
    HPRMS_FILL_SHAPES(HPRMS_FUSED_ENTRY, HPRMS_DTYPE_BF16, 0)
    HPRMS_XCD_ORDER_SHAPES(HPRMS_FUSED_ENTRY, HPRMS_DTYPE_BF16, 0)
    HPRMS_SHAPE_CANDIDATES(HPRMS_FUSED_ENTRY, HPRMS_DTYPE_BF16, 0)
    HPRMS_ALT_ORDER_SHAPES(HPRMS_FUSED_ENTRY, HPRMS_DTYPE_BF16, 0)
    HPRMS_STREAM_POLICY_SHAPES(HPRMS_FUSED_ENTRY, HPRMS_DTYPE_BF16, 0)
    HPRMS_SHARED_UNPACK_SHAPES(HPRMS_FUSED_ENTRY, HPRMS_DTYPE_BF16, 0)
    HPRMS_QUANT_RUNS_AB(HPRMS_FUSED_ENTRY, HPRMS_DTYPE_BF16)
#endif
};

bool entry_is(const FusedEntry& e, int dtype, int mode, const hprms_config& c) {
  return e.dtype == dtype && e.mode == mode && e.lpr == c.lanes_per_row && e.vpl == c.vec_per_lane &&
         e.ldsv == c.lds_vec_per_lane && e.block == c.block_threads && e.flags == c.flags;
}

// the three registries: the aligned kernels, the unaligned and the tail variants
struct Registry {
  const FusedEntry* entries;
  int count;
};
const Registry kRegistries[] = {{kFused, (int)(sizeof(kFused) / sizeof(kFused[0]))},
                                {kFusedUnaligned, kFusedUnalignedCount},
                                {kFusedTail, kFusedTailCount}};

// Each registry holds one kind of variant, told apart by flags bits 5 and 6,
// so a lookup scans only the registry the configuration belongs to.
const FusedEntry* find_fused(int dtype, int mode, const hprms_config& c) {
  const Registry& r = kRegistries[(c.flags & 64) ? 2 : (c.flags & 32) ? 1 : 0];
  for (int i = 0; i < r.count; ++i)
    if (entry_is(r.entries[i], dtype, mode, c)) return &r.entries[i];
  return nullptr;
}

// ---- compute units ------------------------------------------------------------------
// The table's row-count rules (below) were measured on a whole MI355X, 256 CUs.
// What they depend on is rows per CU, so on a device with another count (a
// partition of an MI355X, say) each rule sees the equivalent row count on 256
// CUs, rows * 256 / CUs rounded up; rounds of workgroups are counted on the
// device's own CUs.  (The reference sizes its persistent grid from the
// device's multiProcessorCount, hp_rms_norm/csrc/cuda/hp_rms_norm.cuh:550.)
constexpr int kRefCUs = 256;
constexpr int kMaxDevices = 64;
// CUs per device ordinal, 0 until queried.  Threads that race on a first query
// store the same value.
std::atomic<int> g_cus[kMaxDevices];

// CUs of device `dev` (queried once per ordinal), or a negative status
int device_cus(int dev) {
  if (dev >= 0 && dev < kMaxDevices) {
    const int n = g_cus[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
  }
  int n = 0;
  const hipError_t e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess || n < 1) {
    (void)hipGetLastError();  // not left for the next launch check to report
    return fail(HPRMS_E_LAUNCH, "CU count of device %d: %s", dev,
                e != hipSuccess ? hipGetErrorString(e) : "no compute units reported");
  }
  if (dev >= 0 && dev < kMaxDevices) g_cus[dev].store(n, std::memory_order_relaxed);
  return n;
}

// CUs of the current device; 256 when there is no device to ask (a launch
// would then fail and report why)
int current_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return kRefCUs;
  }
  const int n = device_cus(dev);
  return n > 0 ? n : kRefCUs;
}

// ---- batch-invariant mode -----------------------------------------------------------
// The row-count rules below pick, for one width, shapes whose lanes sum a
// row's squares in different orders, so a row's output can differ by an ulp
// between calls of different row counts.  In batch-invariant mode the shape
// follows from the width, the dtype, the form and the layout alone (the
// bandwidth table's choice for a large batch), as the reference's does
// (hp_rms_norm/csrc/cuda/hp_rms_norm.cuh:562-618), and the row's bits do not
// depend on the call's row count.  Process-wide: -1 until first read, then
// HPRMS_BATCH_INVARIANT from the environment ("1" turns it on) unless set
// through hprms_set_batch_invariant; threads racing on the first read store
// the same value.
std::atomic<int> g_batch_invariant{-1};

bool batch_invariant() {
  int v = g_batch_invariant.load(std::memory_order_relaxed);
  if (v < 0) {
    const char* e = getenv("HPRMS_BATCH_INVARIANT");
    v = (e && e[0] == '1' && e[1] == '\0') ? 1 : 0;
    int expected = -1;
    g_batch_invariant.compare_exchange_strong(expected, v, std::memory_order_relaxed);
    v = g_batch_invariant.load(std::memory_order_relaxed);
  }
  return v == 1;
}

// the row count the table sees in batch-invariant mode: past every row-count rule
constexpr int64_t kInvariantRows = int64_t(1) << 30;

// `rows` on a device of `cus` CUs as the row count with as many rows per CU on 256
int64_t rows_at_ref(int64_t rows, int cus) {
  if (cus == kRefCUs || rows > (int64_t(1) << 40)) return rows;
  return (rows * kRefCUs + cus - 1) / cus;
}

// ---- the gfx950 table -------------------------------------------------------------
// Chosen from (rows, hidden) by measurement on MI355X.  With few rows the
// kernel is latency-bound: one row per workgroup and at most two vectors per
// lane shortens each wave's serial work.  Up to 2048 elements the weight is
// loaded together with the row: a one- or two-wave row then waits for one
// memory round trip instead of two (H = 1024: 2.4-4.5% faster for the fused,
// out-of-place and MX forms, 1-256 rows, hot and cold; H = 2048: up to 1.2%).
// From 4096 up, loading it after the row's sum measured as fast or faster.
//
// These rows stay ahead of the bandwidth table well past one row per CU, by
// how much depending on the mode, so the largest row count that still takes
// them is set per mode (two builds of the library timed side by side, 8
// interleaved trials, 320-1536 rows, hot and cold): the fused op gains 2-29% up to 768-1024 rows at
// H <= 4096 and 37-62% with its rows cache-resident at 8K-16K up to 384
// (within 2% cold); plain RMSNorm 8-36% at H <= 1024 and 2K-4K, the FP8 and MX
// outputs 2-23%.  The out-of-place and partial-sum forms were faster at some
// row counts and up to 15% slower at others, so they keep one row per CU.
// Otherwise the bandwidth table below applies.
bool latency_config(int64_t rows, int64_t nvec, int mode, hprms_config* c) {
  if (nvec <= 64 || nvec > 2048) return false;
  struct Row { int64_t max_nvec; int lpr, vpl; };
  static const Row lat[] = {{128, 64, 2}, {256, 128, 2}, {512, 256, 2}, {1024, 512, 2}, {2048, 512, 4}};
  // most rows that take each latency row: fused; plain; FP8 and MX; out of place and partial sums
  static const int16_t max_rows[4][5] = {{1024, 768, 768, 256, 384},
                                         {1024, 256, 768, 256, 256},
                                         {1024, 768, 768, 256, 256},
                                         {256, 256, 256, 256, 256}};
  const int cls = mode == 0 ? 0 : mode == 1 ? 1 : (mode == 2 || mode >= 5) ? 2 : 3;
  for (int i = 0; i < 5; ++i) {
    const Row& r = lat[i];
    if (nvec <= r.max_nvec) {
      if (rows > max_rows[cls][i]) return false;
      // (the partial sums load all their parts before adding them: flags bit 15)
      *c = hprms_config{1, r.lpr, r.vpl, 0, r.lpr, 0, (nvec <= 256 ? 3 : 7) | (mode == 4 ? 32768 : 0)};
      return true;
    }
  }
  return false;
}

// The FP8 output adds a second row reduction (the absolute maximum) and a
// barrier; at 1K < H <= 2K it prefers two vectors per lane, one row per
// 128-lane workgroup (5-9% faster than the fused table's 64 x 4 at 4096 rows,
// as for the MX outputs, 5-11%); from 3K elements more, smaller workgroups per CU, and
// at 32K the LDS tier (measured 5.8% faster than 1024 lanes x 4 in registers),
// with the residual's loads first (1-1.9% faster at 25K-32K).
bool fp8_config(int64_t nvec, hprms_config* c) {
  struct Row { int64_t min_nvec, max_nvec; int lpr, vpl, ldsv, block, flags; };
  static const Row fp8[] = {{129, 256, 128, 2, 0, 128, 3},
                            {385, 512, 256, 2, 0, 256, 7},
                            {513, 640, 256, 3, 0, 256, 7},
                            {641, 1024, 512, 2, 0, 512, 7},
                            {1537, 2048, 1024, 2, 0, 1024, 31},
                            {3073, 4096, 512, 8, 4, 512, 159}};
  for (const Row& r : fp8) {
    if (nvec >= r.min_nvec && nvec <= r.max_nvec) {
      *c = hprms_config{r.ldsv > 0 ? 2 : 1, r.lpr, r.vpl, r.ldsv, r.block, 0, r.flags};
      return true;
    }
  }
  return false;
}

// The MX outputs (per-block maxima: a DPP quad step, no second barrier)
// measured best with the register tier at 32K (1024 x 4: 4.5% / 5% faster
// than the FP8 table's LDS tier for MXFP8 / MXFP4) and with 256 lanes x 2 at
// 3K < H <= 4K.
bool mx_config(int64_t nvec, hprms_config* c) {
  struct Row { int64_t min_nvec, max_nvec; int lpr, vpl, ldsv, block, flags; };
  static const Row mx[] = {{129, 256, 128, 2, 0, 128, 3},
                           {385, 512, 256, 2, 0, 256, 7},
                           {513, 640, 256, 3, 0, 256, 7},
                           {641, 1024, 512, 2, 0, 512, 7},
                           {1537, 2048, 1024, 2, 0, 1024, 31},
                           {3073, 4096, 1024, 4, 0, 1024, 159}};
  for (const Row& r : mx) {
    if (nvec >= r.min_nvec && nvec <= r.max_nvec) {
      *c = hprms_config{1, r.lpr, r.vpl, r.ldsv, r.block, 0, r.flags};
      return true;
    }
  }
  return false;
}

// At 4K < H <= 5K plain RMSNorm, the FP8 and the MX outputs take 256 lanes x 3
// vectors (512 x 2 leaves half its lanes idle there): plain 2.5-7.3%, FP8 1-4%,
// MX 0.3-2.6% faster (two builds side by side, 4096 rows); the fused op
// measured 0.8-1.5% slower with it and keeps 512 x 2.
//
// Plain RMSNorm moves half the bytes of the fused op per row and has no
// residual phase; measured against the fused table it prefers one wave per row
// at 2K < H <= 4K (10-14% faster, no barrier), 512 lanes up to 8K and at
// 12K-16K (2-3%), and 512 lanes x 8 vectors at 24K-32K (4-8%).
bool plain_config(int64_t nvec, hprms_config* c) {
  struct Row { int64_t min_nvec, max_nvec; int lpr, vpl, block, flags; };
  static const Row plain[] = {{257, 512, 64, 8, 256, 3},
                              {513, 640, 256, 3, 256, 7},
                              {641, 1024, 512, 2, 512, 31},
                              {1537, 2048, 512, 4, 512, 31},
                              {3073, 4096, 512, 8, 512, 7}};
  for (const Row& r : plain) {
    if (nvec >= r.min_nvec && nvec <= r.max_nvec) {
      *c = hprms_config{1, r.lpr, r.vpl, 0, r.block, 0, r.flags};
      return true;
    }
  }
  return false;
}

// The in-place op (mode 0) on rows on the 128-byte grid takes one row per
// 256-lane workgroup at 3K < H <= 4K: 256 lanes x 2 vectors, 0.9-1.8% faster
// than 128 x 4 with two rows per workgroup (interleaved cold trials at 4096
// rows, five runs, H = 3584 and 4096).  Rows off the grid keep 128 x 4: with
// one row per workgroup every cache line two neighbouring rows share is
// written by two workgroups, and its variants measured 13-18% slower (4096
// rows at H = 4097, and at H = 4096 with rows 2 bytes off).  The out-of-place
// and partial-sum forms keep the shared row.
bool inplace_config(int64_t nvec, hprms_config* c) {
  if (nvec <= 384 || nvec > 512) return false;
  *c = hprms_config{1, 256, 2, 0, 256, 0, 131};
  return true;
}

// The partial-sum form reads P + 1 rows per output row; at 4K < H <= 8K it
// measured 1.3-5.8% faster with 256 lanes x 4 than with the fused table's
// 512 x 2 (which the fused and out-of-place forms prefer by 0.2-2.1%).
bool reduce_config(int64_t nvec, hprms_config* c) {
  if (nvec <= 512 || nvec > 1024) return false;
  *c = hprms_config{1, 256, 4, 0, 256, 0, 3};
  return true;
}

// The table's 1024 x 2 and 1024 x 3 rows (12K < H <= 24.5K) load the weight
// together with the row in the fused op and its out-of-place and partial-sum
// forms (modes 0, 3, 4): 0.8-1.6% faster (bf16 and fp16, on the 128-byte grid
// and rotated off it; 4096 rows, two builds side by side, 9 interleaved
// trials; one row: 2% slower).  Plain RMSNorm measured the same either way;
// the FP8 and MX outputs ran 12-23% slower with it and the tail variants
// 2-4% (tail_shape): they load it late.
bool weight_late_1024(int mode, const hprms_config& c) {
  if (c.lanes_per_row != 1024 || (c.vec_per_lane != 2 && c.vec_per_lane != 3)) return false;
  return !(mode == 0 || mode == 3 || mode == 4);
}

// Rows of 1K-3K (128 < H / 8 <= 384) in the fused op in and out of place,
// 1024 < rows <= 4096: 32 lanes x ceil(H / 256) vectors, two rows per one-wave
// workgroup (flags 135: residual first, weight late), in place of the table's
// 128 x 3 (2K-3K) and, where its last round of workgroups leaves CUs idle or
// past 3072 rows, of its 64 x 4 (four rows per 256-lane workgroup, 1K-2K).
// Two builds side by side, 7 interleaved trials, both dtypes: at 1K-2.5K
// 5-15% faster at 1280-1536, 2304-2560 and 3584-4096 rows and at 2048-3072
// rows past 2K, within 3% at 1280 rows past 2K; at 2.5K-3K 7-16% faster at
// 1536-4096 rows (4096 x 3072 bf16: 18.07 -> 16.66 us) but 3-7% slower for
// fp16 in place at 4096 rows (2816, and rows off the 128-byte grid); at
// 1280-1536 rows 8-14% faster out of place, 0-6% slower in place (which
// keeps the table there).  Kept out of: 64 x 4 with even
// rounds at 1024 / 1792-2048 / 3072 rows (0-16% slower), 1024 rows and fewer
// (up to 27% slower out of place), 5120 rows and more (fp16 and the
// out-of-place op up to 14% slower, 32 x 11 and x 12 6-8% at 8192 rows), and
// past 3K, where 32 x 13 and x 14 need the whole register file in some forms
// (one wave per SIMD: 2-7% slower there; held to two waves they spill).
// Eight rows per 256-lane workgroup, and the FP8, MX and partial-sum forms,
// measured slower with the wider rows.
// (`r`: the row count scaled to 256 CUs, rows_at_ref; `rows` and `cus`: the
// call's own, for the rounds of workgroups.)
//
// rows per CU with `rows_per_wg` rows per workgroup, whole rounds of workgroups
int64_t rows_per_cu(int64_t rows, int64_t rows_per_wg, int cus) {
  return ((rows + rows_per_wg - 1) / rows_per_wg + cus - 1) / cus * rows_per_wg;
}

bool wide_rows(int64_t rows, int64_t r, int64_t nvec, int mode, int cus) {
  if ((mode != 0 && mode != 3) || nvec <= 128 || nvec > 384 || r <= 1024 || r > 4096) return false;
  if (nvec > 320) return mode == 3 || r > 1536;
  return nvec > 256 || r > 3072 || rows_per_cu(rows, 2, cus) < rows_per_cu(rows, 4, cus);
}

// Rows of 3K-5K (384 < H / 8 <= 640) in the fused op in and out of place and
// in plain RMSNorm (8-32% faster, both dtypes; the FP8 output measured 1-11%
// slower) on the 128-byte grid, 768 < rows <= 2048: one row per one-wave
// workgroup, 64
// lanes x ceil(H / 512) vectors (flags 135), in place of the table's 256 x 2
// / 128 x 4 and 512 x 2.  Two builds side by side, 7 interleaved trials, both
// dtypes, H = 3584-5120: in place 2-18% faster at 769-2048 rows (1024 x 4096
// bf16: 7.36 -> 6.43 us), out of place 3-20%; out of place at 300-512 rows
// 0-12% slower; with forced shapes 1-5% faster at 2560-3072 rows and 3%
// slower at 4096.  Past 5K the fp16 kernels need the whole register file
// (64 x 12: one wave per SIMD) and lost 2-7% at 2048 rows.  Rows off the grid
// keep the table (inplace_config: two rows per workgroup).
bool wave_rows(int64_t rows, int64_t nvec, int mode, bool grid) {
  return (mode == 0 || mode == 1 || mode == 3) && grid && nvec > 384 && nvec <= 640 && rows > 768 && rows <= 2048;
}

// Rows of 5K-8K (640 < H / 8 <= 1024) in the fused op in and out of place on
// the 128-byte grid, 512 < rows <= 1280: one row per two-wave workgroup, 128
// lanes x ceil(H / 1024) vectors (flags 135), in place of the table's 512 x 2
// (one row per 8-wave workgroup).  Two builds side by side, 7 interleaved
// trials, H = 5632-8192: in place 2-14% faster (bf16; 1024 x 6144: 10.26 ->
// 9.07 us), out of place 3-18%; fp16 at 513 x 7-8K 2-5% slower.  Forced
// shapes: 3-14% slower at 300 rows, -2% to +7% at 1536-2560 rows.
bool pair_rows(int64_t rows, int64_t nvec, int mode, bool grid) {
  return (mode == 0 || mode == 3) && grid && nvec > 640 && nvec <= 1024 && rows > 512 && rows <= 1280;
}

// `grid`: every row of every stream starts on the 128-byte grid (only the
// in-place op's rows depend on it); `cus`: the device's compute units.
void table_config(int64_t rows, int64_t hidden, int mode, bool grid, int cus, hprms_config* c) {
  if (batch_invariant()) rows = kInvariantRows;
  const int64_t nvec = hidden / 8;
  const int64_t r = rows_at_ref(rows, cus);
  if (latency_config(r, nvec, mode, c)) return;
  if (wide_rows(rows, r, nvec, mode, cus)) {
    *c = hprms_config{1, 32, (int)((nvec + 31) / 32), 0, 64, 0, 135};
    return;
  }
  if (wave_rows(r, nvec, mode, grid)) {
    *c = hprms_config{1, 64, (int)((nvec + 63) / 64), 0, 64, 0, 135};
    return;
  }
  if (pair_rows(r, nvec, mode, grid)) {
    *c = hprms_config{1, 128, (int)((nvec + 127) / 128), 0, 128, 0, 135};
    return;
  }
  if (mode == 0 && grid && inplace_config(nvec, c)) return;
  if (mode == 1 && plain_config(nvec, c)) return;
  if (mode == 4 && reduce_config(nvec, c)) return;
  if (mode == 2 && fp8_config(nvec, c)) return;
  if (mode >= 5 && mx_config(nvec, c)) return;   // MX and the FP8 output with a scale per 128 elements
  *c = hprms_config{1, 0, 0, 0, 0, 0, 3};
  // flags: 3 = non-temporal row loads and stores, +4 = weight loaded late,
  // +24 = sc1 on loads and stores, +128 = residual loads before input loads
  // (9K-12K: 0.4-0.6% faster with them, interleaved cold trials)
  struct Row { int64_t max_nvec; int lpr, vpl, ldsv, block, flags; };
  static const Row table[] = {
      {16, 16, 1, 0, 256, 3},        // H <= 128:   16 rows per workgroup
      {32, 32, 1, 0, 256, 3},        // H <= 256
      {64, 64, 1, 0, 256, 3},        // H <= 512:   one row per wave
      {128, 32, 4, 0, 256, 131},     // H <= 1024:  two rows per wave
      {256, 64, 4, 0, 256, 135},     // H <= 2048
      {384, 128, 3, 0, 256, 7},      // H <= 3072:  two waves per row
      {512, 128, 4, 0, 256, 131},    // H <= 4096
      {1024, 512, 2, 0, 512, 7},     // H <= 8192:  one row per 8-wave workgroup
      {1536, 512, 3, 0, 512, 159},   // H <= 12288
      {2047, 1024, 2, 0, 1024, 27},  // H <= 16376
      {2048, 256, 8, 4, 256, 27},    // H = 16384: LDS tier, half the row in LDS
      {3072, 1024, 3, 0, 1024, 155}, // H <= 24576
      {4096, 1024, 4, 0, 1024, 159}, // H <= 32768
      {8192, 1024, 8, 4, 1024, 31},  // H <= 65536: LDS tier
  };
  for (const Row& r : table) {
    if (nvec <= r.max_nvec) {
      c->lanes_per_row = r.lpr;
      c->vec_per_lane = r.vpl;
      c->lds_vec_per_lane = r.ldsv;
      c->block_threads = r.block;
      c->flags = r.flags;
      c->tier = r.ldsv > 0 ? 2 : 1;
      if (weight_late_1024(mode, *c)) c->flags |= 4;
      return;
    }
  }
  c->tier = 3;
  c->lanes_per_row = 256;
  c->block_threads = 256;
}

// Row groups in runs per XCD (hprms_device.h, xcd_runs; flags bits 16-18 =
// V: each XCD takes 2^V consecutive row groups in place of every 8th).  The
// in-place op on rows on the 128-byte grid whose input and residual share a
// row pitch in this table, with the table's kernel for that pitch, measured
// faster this way (bf16, cold, interleaved trials, repeated on fresh boxes):
// 8 KiB rows (H = 4096) with runs of 32, 0.6-1.1% at 4096-16384 rows; 16 KiB
// (H = 8192) with runs of 64, 1.1-1.9% at 2048-8192 rows (0.4% at 16384).
// At the other 17 widths of the benchmark sweep (4096 rows) every run length
// from 2 to 128 was as fast or slower (up to 16%) or less than 1% faster
// (56 KiB, H = 28672: runs of 8, 0.2-1.0% at 2048-16384 rows; left out), and
// at 64 KiB (H = 32768) runs of 8 ranged from 3.6% faster to 4% slower with
// the row count.  The order only changes which workgroup takes a row, so the
// bits are the same.
// The quantised outputs (modes 2, 5, 6, 7) at 16 KiB rows with their table
// kernel (512 x 2), runs of 32: 0.3-1.1% faster at 4096 rows (seven
// interleaved trials), and 5.7% for mode 7 with column-major scales.  Those
// scales are 4-byte stores, 32 rows to a 128-byte line; with one row per
// workgroup the 32 rows of a line otherwise go to all 8 XCDs, and each XCD's
// L2 writes its part of the line back on its own.  Mode 7 with column-major
// scales also takes runs of 32 at 8 KiB rows (256 x 2): 2.2-3.5% faster;
// there modes 2, 5 and 6 were within 0.4% either way, and mode 7 with rows
// of scales from 1.1% faster to 0.5% slower over two boxes, so left out.  At
// 32 and 64 KiB rows (1024 lanes, one row per workgroup) runs of 8-64 were
// 3-13% slower in mode 7.
struct RunsRow {
  unsigned modes;       // bit m: mode m
  bool scale_columns;   // mode 7 with column-major scales only
  int64_t pitch_bytes;
  int lpr, vpl, block, flags, v;
  int64_t min_rows;  // on 256 CUs
};
constexpr unsigned kQuantModes = 1u << 2 | 1u << 5 | 1u << 6 | 1u << 7;
constexpr RunsRow kRuns[] = {{1u, false, 8192, 256, 2, 256, 131, 5, 4096},
                             {1u, false, 16384, 512, 2, 512, 7, 6, 2048},
                             {kQuantModes, false, 16384, 512, 2, 512, 7, 5, 4096},
                             {1u << 7, true, 8192, 256, 2, 256, 7, 5, 4096}};

// flags bits 16-18 for configuration c of mode `mode` on rows `pitch_bytes`
// apart in both input streams, on the 128-byte grid (scale_columns: mode 7's
// scales are column-major); 0 for others
int xcd_runs_flags(int mode, int64_t rows, int64_t pitch_bytes, int cus, const hprms_config& c,
                   bool scale_columns) {
  if (c.tier != 1 || c.lds_vec_per_lane != 0) return 0;
  for (const RunsRow& r : kRuns)
    if (((r.modes >> mode) & 1u) && (!r.scale_columns || scale_columns) && r.pitch_bytes == pitch_bytes &&
        r.lpr == c.lanes_per_row && r.vpl == c.vec_per_lane && r.block == c.block_threads && r.flags == c.flags &&
        rows_at_ref(rows, cus) >= r.min_rows)
      return r.v << 16;
  return 0;
}

constexpr int64_t kMaxHidden = int64_t(1) << 24;
constexpr int64_t kMaxGrid = 0x7fffffff;

struct Problem {
  int mode;  // 0 fused, 1 plain, 2 fused with FP8 output, 3 fused out of place, 4 parts reduced first,
             // 5 / 6 MX output, 7 FP8 output with a scale per 128 elements
  void* x;    // mode 4: parts[0]
  void* out;  // modes 1, 3, 4: 16-bit output; mode 2: FP8 output
  void* res;
  const void* w;
  int64_t rows, hidden, x_stride, out_stride, res_stride;
  int dtype;
  double eps;
  float* scale = nullptr;      // mode 2: per-row scales, written
  const float* static_scale = nullptr;  // mode 2: one given scale for every row (then no `scale`)
  const float* scale_ub = nullptr;      // mode 2, per-row scales: upper bound on the row maximum
  void* res_out = nullptr;     // mode 3
  int64_t res_out_stride = 0;  // mode 3
  int nparts = 1;              // mode 4
  const void* const* parts = nullptr;
  void* mx_scales = nullptr;   // modes 5, 6: E8M0 bytes; mode 7: float32
  int64_t mx_scale_stride = 0; // bytes
  int64_t mx_group_stride = 4; // mode 7: bytes between a row's consecutive scales
  int64_t* timeline = nullptr; // configurations with flags bit 9 (bench library)
};

bool is_mx(int mode) { return mode == 5 || mode == 6; }
// outputs with per-block scales: the MX modes (one E8M0 byte per 32 elements)
// and mode 7 (one float32 per 128 elements); either way hidden / 32 scale
// bytes per row
bool is_blockq(int mode) { return is_mx(mode) || mode == 7; }

// Mode 7's scale (row r, group g) sits at byte r * mx_scale_stride + g *
// mx_group_stride.  Bytes one row's scales span: (groups - 1) * group stride
// + 4 (hidden / 32 for rows of scales).
int64_t group_extent(const Problem& p) { return (p.hidden / 128 - 1) * p.mx_group_stride + 4; }

// The scales form rows (each row's groups inside the gap to the next row) or
// columns (each group's rows inside the gap to the next group), so no two
// (row, group) pairs share a scale; interleaved layouts are refused.  Strides in bytes, at most 2^42 (the entry
// point's bound), groups at most kMaxHidden / 128 = 2^17, so no product
// here passes 2^59.
bool group_scales_disjoint(const Problem& p) {
  const int64_t groups = p.hidden / 128, rs = p.mx_scale_stride, gs = p.mx_group_stride;
  if (rs < 0 || gs < 0) return false;
  const bool rows_of_scales = (groups <= 1 || gs >= 4) && (p.rows <= 1 || rs >= (groups - 1) * gs + 4);
  // (rows - 1) * rs + 4 <= gs <= 2^42, so rows past 2^42 / rs never fit
  const bool columns = (p.rows <= 1 || rs >= 4) &&
                       (groups <= 1 || (p.rows - 1 <= (int64_t(1) << 42) / (rs > 0 ? rs : 1) &&
                                        gs >= (p.rows - 1) * rs + 4));
  return rows_of_scales || columns;
}
// bytes of quantised output per row (modes 2, 5, 6)
int64_t q_row_bytes(int mode, int64_t hidden) { return mode == 6 ? hidden / 2 : hidden; }

bool has_res(int mode) { return mode != 1; }
bool has_out(int mode) { return mode != 0; }

// No buffer on any GPU spans more bytes (virtual addresses have at most 57
// bits), and under this bound the kernels' 64-bit row offsets cannot overflow.
constexpr int64_t kMaxExtentBytes = int64_t(1) << 56;

// `rows` rows of `width` elements of `elem` bytes, `stride` elements apart,
// span at most kMaxExtentBytes
bool extent_ok(int64_t rows, int64_t stride, int64_t elem, int64_t width) {
  if (rows <= 1) return true;
  if (stride > kMaxExtentBytes / elem) return false;
  return rows - 1 <= (kMaxExtentBytes / elem - width) / stride;
}

int check_problem(const Problem& p) {
  if (p.dtype != HPRMS_DTYPE_BF16 && p.dtype != HPRMS_DTYPE_FP16)
    return fail(HPRMS_E_INVALID, "dtype must be HPRMS_DTYPE_BF16 or HPRMS_DTYPE_FP16 (got %d)", p.dtype);
  if (p.rows < 0) return fail(HPRMS_E_INVALID, "rows must be >= 0 (got %lld)", (long long)p.rows);
  if (p.hidden < 1) return fail(HPRMS_E_INVALID, "hidden must be >= 1 (got %lld)", (long long)p.hidden);
  if (p.hidden > kMaxHidden)
    return fail(HPRMS_E_RANGE, "hidden %lld exceeds the supported maximum %lld", (long long)p.hidden,
                (long long)kMaxHidden);
  if (p.x_stride < p.hidden) return fail(HPRMS_E_INVALID, "input row stride %lld < hidden %lld",
                                         (long long)p.x_stride, (long long)p.hidden);
  if (has_res(p.mode) && p.res_stride < p.hidden)
    return fail(HPRMS_E_INVALID, "residual row stride %lld < hidden %lld", (long long)p.res_stride,
                (long long)p.hidden);
  if (is_mx(p.mode) && p.hidden % 32 != 0)
    return fail(HPRMS_E_INVALID, "MX output needs hidden %% 32 == 0 (got %lld)", (long long)p.hidden);
  if (p.mode == 7 && p.hidden % 128 != 0)
    return fail(HPRMS_E_INVALID, "FP8 output with a scale per 128 elements needs hidden %% 128 == 0 (got %lld)",
                (long long)p.hidden);
  if (has_out(p.mode) && p.out_stride < q_row_bytes(p.mode, p.hidden))
    return fail(HPRMS_E_INVALID, "output row stride %lld < %lld", (long long)p.out_stride,
                (long long)q_row_bytes(p.mode, p.hidden));
  if (is_mx(p.mode) && p.mx_scale_stride < p.hidden / 32)
    return fail(HPRMS_E_INVALID, "scale row stride %lld < hidden / 32 = %lld", (long long)p.mx_scale_stride,
                (long long)(p.hidden / 32));
  if (p.mode == 7 && !group_scales_disjoint(p))
    return fail(HPRMS_E_INVALID,
                "scale strides (row %lld, group %lld) lay the scales out neither as rows (row stride > "
                "(hidden / 128 - 1) * group stride, group stride >= 1) nor as columns (group stride > "
                "(rows - 1) * row stride, row stride >= 1)",
                (long long)(p.mx_scale_stride / 4), (long long)(p.mx_group_stride / 4));
  if (p.mode == 3 && p.res_out_stride < p.hidden)
    return fail(HPRMS_E_INVALID, "residual output row stride %lld < hidden %lld", (long long)p.res_out_stride,
                (long long)p.hidden);
  if (p.mode == 4 && (p.nparts < 1 || p.nparts > HPRMS_MAX_PARTS))
    return fail(HPRMS_E_INVALID, "nparts must be in [1, %d] (got %d)", HPRMS_MAX_PARTS, p.nparts);
  if (!(p.eps >= 0.0)) return fail(HPRMS_E_INVALID, "eps must be >= 0");
  if (p.rows == 0) return HPRMS_OK;
  const int64_t ob = (p.mode == 2 || is_blockq(p.mode)) ? 1 : 2;  // bytes per output element
  if (!extent_ok(p.rows, p.x_stride, 2, p.hidden) ||
      (has_res(p.mode) && !extent_ok(p.rows, p.res_stride, 2, p.hidden)) ||
      (has_out(p.mode) && !extent_ok(p.rows, p.out_stride, ob, q_row_bytes(p.mode, p.hidden))) ||
      (p.mode == 3 && !extent_ok(p.rows, p.res_out_stride, 2, p.hidden)) ||
      (is_mx(p.mode) && !extent_ok(p.rows, p.mx_scale_stride, 1, p.hidden / 32)) ||
      (p.mode == 7 && !extent_ok(p.rows, p.mx_scale_stride, 1, group_extent(p))))
    return fail(HPRMS_E_RANGE, "%lld rows at these row strides span more than 2^56 bytes", (long long)p.rows);
  if (p.mode == 4 && !p.parts) return fail(HPRMS_E_INVALID, "null parts array");
  if (!p.x || !p.w || (has_res(p.mode) && !p.res) || (has_out(p.mode) && !p.out) ||
      (p.mode == 2 && !p.scale && !p.static_scale) ||
      (p.mode == 3 && !p.res_out) || (is_blockq(p.mode) && !p.mx_scales))
    return fail(HPRMS_E_INVALID, "null tensor pointer");
  if (p.mode == 7 && ((uintptr_t)p.mx_scales & 3u) != 0)
    return fail(HPRMS_E_INVALID, "the float32 scales must be 4-byte aligned");
  if (p.mode == 4) {
    for (int g = 0; g < p.nparts; ++g) {
      if (!p.parts[g]) return fail(HPRMS_E_INVALID, "null tensor pointer (part %d)", g);
      if (p.parts[g] == p.res) return fail(HPRMS_E_INVALID, "part %d and residual must not alias", g);
    }
    if (p.out == p.res) return fail(HPRMS_E_INVALID, "output and residual must not alias");
    for (int g = 0; g < p.nparts; ++g)
      if (p.parts[g] == p.out && p.out_stride != p.x_stride)
        return fail(HPRMS_E_INVALID, "output aliases part %d with a different row stride", g);
    return HPRMS_OK;
  }
  if (p.mode == 3) {
    if (p.out == p.res_out) return fail(HPRMS_E_INVALID, "output and residual output must not alias");
    if (p.out == p.res || p.res_out == p.x)
      return fail(HPRMS_E_INVALID, "output and residual output may only alias input and residual respectively");
    if ((p.out == p.x && p.out_stride != p.x_stride) || (p.res_out == p.res && p.res_out_stride != p.res_stride))
      return fail(HPRMS_E_INVALID, "an in-place alias needs equal row strides");
    return HPRMS_OK;
  }
  if (has_res(p.mode) && p.x == p.res) return fail(HPRMS_E_INVALID, "input and residual must not alias");
  return HPRMS_OK;
}

// Can the vector tiers take this problem with configuration c?  The
// unaligned variants (flags bit 5) take rows at any 2-byte boundary, and with
// the tail (bit 6) any hidden >= 8; the others need 16-byte aligned rows.
// Without the tail, hidden % 8 == 0.
bool vec_fits(const Problem& p, const hprms_config& c) {
  if ((c.flags & 64) ? p.hidden < 8 : p.hidden % 8 != 0) return false;  // the tail overlaps a whole vector
  if (c.flags & 32) {
    if (!aligned2(p.x) || !aligned2(p.w)) return false;
    if (has_res(p.mode) && !aligned2(p.res)) return false;
    if ((p.mode == 1 || p.mode == 3 || p.mode == 4) && !aligned2(p.out)) return false;
    if (p.mode == 3 && !aligned2(p.res_out)) return false;
    if (p.mode == 4 && p.parts)  // null only with rows == 0 (a configuration check)
      for (int g = 0; g < p.nparts; ++g)
        if (!aligned2(p.parts[g])) return false;
  } else {
    if (!aligned16(p.x) || !aligned16(p.w)) return false;
    if (p.x_stride % 8 != 0) return false;
    if (has_res(p.mode) && (!aligned16(p.res) || p.res_stride % 8 != 0)) return false;
    if (p.mode == 2 || p.mode == 5 || p.mode == 7) {
      if (((uintptr_t)p.out & 7u) != 0 || p.out_stride % 8 != 0) return false;
    } else if (p.mode == 6) {
      if (((uintptr_t)p.out & 3u) != 0 || p.out_stride % 4 != 0) return false;
    } else if (has_out(p.mode) && (!aligned16(p.out) || p.out_stride % 8 != 0)) {
      return false;
    }
    if (p.mode == 3 && (!aligned16(p.res_out) || p.res_out_stride % 8 != 0)) return false;
    if (p.mode == 4 && p.parts)
      for (int g = 0; g < p.nparts; ++g)
        if (!aligned16(p.parts[g])) return false;
  }
  if ((int64_t)c.lanes_per_row * c.vec_per_lane < p.hidden / 8) return false;  // whole vectors
  // the kernels take the input and residual (plain RMSNorm: output) row strides as 32-bit scalars
  if (p.x_stride > INT32_MAX || (has_res(p.mode) && p.res_stride > INT32_MAX)) return false;
  if (p.mode == 1 && p.out_stride > INT32_MAX) return false;
  // every buffer resource of a row group spans < 2^31 bytes
  const int64_t rpb = c.block_threads / c.lanes_per_row;
  int64_t smax = p.x_stride > p.out_stride ? p.x_stride : p.out_stride;
  if (has_res(p.mode) && p.res_stride > smax) smax = p.res_stride;
  if (p.mode == 3 && p.res_out_stride > smax) smax = p.res_out_stride;
  // the MX scale rows have their own buffer resource (byte stride)
  if (is_mx(p.mode) && (rpb - 1) * p.mx_scale_stride + p.hidden / 32 >= (int64_t)kOOB) return false;
  if (p.mode == 7 && (rpb - 1) * p.mx_scale_stride + group_extent(p) >= (int64_t)kOOB) return false;
  // a 128-element group of mode 7 is 16 adjacent lanes' vectors
  if (p.mode == 7 && c.lanes_per_row % 16 != 0) return false;
  if (((rpb - 1) * smax + p.hidden) * 2 + 16 * (int64_t)c.lanes_per_row * c.vec_per_lane >= (int64_t)kOOB)
    return false;
  return true;
}

// Which problems the table sends to the unaligned variant of its shape: rows
// (of any stream) or the weight off the 128-byte grid, or hidden % 8 != 0.
// Rows on the grid keep the measured table entry, sc1 bits included.
bool needs_unaligned(const Problem& p) {
  if (p.hidden % 8 != 0 || ((uintptr_t)p.w & 127u) != 0) return true;
  if (!rows_aligned128(p.x, p.x_stride * 2)) return true;
  if (has_res(p.mode) && !rows_aligned128(p.res, p.res_stride * 2)) return true;
  if (has_out(p.mode)) {
    const bool bytes = p.mode == 2 || is_blockq(p.mode);  // quantised rows: byte strides
    if (!rows_aligned128(p.out, bytes ? p.out_stride : p.out_stride * 2)) return true;
  }
  if (p.mode == 3 && !rows_aligned128(p.res_out, p.res_out_stride * 2)) return true;
  if (p.mode == 4 && p.parts)
    for (int g = 0; g < p.nparts; ++g)
      if (!rows_aligned128(p.parts[g], p.x_stride * 2)) return true;
  return false;
}

// Where a stream's rows start relative to its vector boundaries (16 bytes; 8
// bytes for the FP8 output's byte rows): row r starts (base + r * step) mod 8
// elements past one.
struct Phase {
  uint32_t base, step;
  bool operator==(const Phase& o) const { return base == o.base && step == o.step; }
};
Phase phase16(const void* p, int64_t stride) { return {(uint32_t)(((uintptr_t)p >> 1) & 7u), (uint32_t)(stride & 7)}; }
Phase phase8(const void* p, int64_t stride) { return {(uint32_t)((uintptr_t)p & 7u), (uint32_t)(stride & 7)}; }

// Shifted rows (the tail variant's shift phases), modes 0-4 from 513
// whole vectors up, when no stream of the call (the weight aside: it stays in
// L2) has all its rows on 16-byte boundaries.  The rows are shifted to the
// phase of the first written stream (input / residual in place, the output
// otherwise), which aligns every stream that shares it.  Measured on MI355X
// (4096 rows, bf16, 8K-32K, against the unaligned and unshifted tail
// variants): with every stream off alignment, 6-20% faster in modes 0, 3
// and 4 whether or not the streams share a phase (the least at 16K), and
// 3-34% faster for contiguous rows of odd widths in every mode; shifting an aligned stream off its
// boundaries instead costs 9-39%, so one aligned stream rules the shift out.
// Plain RMSNorm with input and output at different phases shifts only from
// 16K up (up to 5% slower below, 3-10% faster at 24K-32K).  The FP8 output
// shifts only rows of odd widths whose streams share one phase (14-34%
// faster): its byte rows misaligned cost 15-25% at 16K, and for whole-vector
// widths its unaligned variant was as fast or faster.
constexpr int64_t kShiftMinVec = 513;

Phase shift_phase(const Problem& p) {
  const Phase none = {0, 0};
  if (p.mode > 4 || p.hidden / 8 < kShiftMinVec) return none;
  Phase s[4 + HPRMS_MAX_PARTS];
  int n = 0;
  switch (p.mode) {
    case 0:
      s[n++] = phase16(p.x, p.x_stride);
      s[n++] = phase16(p.res, p.res_stride);
      break;
    case 1:
      s[n++] = phase16(p.out, p.out_stride);
      s[n++] = phase16(p.x, p.x_stride);
      break;
    case 2:
      s[n++] = phase16(p.res, p.res_stride);
      s[n++] = phase8(p.out, p.out_stride);
      s[n++] = phase16(p.x, p.x_stride);
      break;
    case 3:
      s[n++] = phase16(p.out, p.out_stride);
      s[n++] = phase16(p.res_out, p.res_out_stride);
      s[n++] = phase16(p.x, p.x_stride);
      s[n++] = phase16(p.res, p.res_stride);
      break;
    default:
      s[n++] = phase16(p.out, p.out_stride);
      s[n++] = phase16(p.res, p.res_stride);
      for (int g = 0; g < p.nparts && p.parts; ++g) s[n++] = phase16(p.parts[g], p.x_stride);
      break;
  }
  bool shared = true;
  for (int i = 0; i < n; ++i) {
    if (s[i] == none) return none;
    if (!(s[i] == s[0])) shared = false;
  }
  if (p.mode == 2) return shared && p.hidden % 8 != 0 ? s[0] : none;
  if (p.mode == 1 && !shared && p.hidden < 16384) return none;
  return s[0];
}

// Rotated rows (the rotation phases of the off-grid variants of modes 0, 1, 3, 4).  With
// rows off the 128-byte grid, a wave's 1 KiB access to a row shares its first
// and last cache line with the neighbouring accesses: such half-written lines
// cost 9-13% against whole ones (a flat two-stream in-place rewrite 16 bytes
// off, 4096 x 4K-32K bf16), and the rows' own measured 10-17% at 16K-32K
// before the rotation.  The kernel rotates each row's lane mapping so that
// every access starts on a 512-byte boundary of one written stream (4096 rows
// at stride H + 8: 0.1-1% faster than 128-byte boundaries at 16K-32K; 1 KiB
// boundaries measured up to 1% faster still, but would make the result's
// bits depend on where torch's allocator, which aligns to 512 bytes, puts a
// buffer): the stream the shift aligns when rows are shifted, otherwise the
// first written stream whose rows are 16-byte aligned but off the 128-byte
// grid, else off the 512-byte grid.  Returns that stream's phase
// {base, step} modulo 512 bytes, or {0, 0} (no rotation).
Phase rot_phase(const Problem& p) {
  const Phase none = {0, 0};
  if (p.mode == 2 || p.mode > 4) return none;
  struct Stream { const void* ptr; int64_t stride; };
  Stream w[2];
  int n = 0;
  switch (p.mode) {
    case 0: w[n++] = {p.x, p.x_stride}; w[n++] = {p.res, p.res_stride}; break;
    case 1: w[n++] = {p.out, p.out_stride}; break;
    case 3: w[n++] = {p.out, p.out_stride}; w[n++] = {p.res_out, p.res_out_stride}; break;
    default: w[n++] = {p.out, p.out_stride}; w[n++] = {p.res, p.res_stride}; break;
  }
  auto phase512 = [](const Stream& s) {
    return Phase{(uint32_t)((uintptr_t)s.ptr & 511u), (uint32_t)((s.stride * 2) & 511)};
  };
  if (p.hidden % 8 != 0 || !(shift_phase(p) == none)) return phase512(w[0]);  // the shifted stream
  // 16-byte aligned rows, not all on a `grid`-byte boundary
  auto off = [](const Stream& s, int grid) {
    return aligned16(s.ptr) && s.stride % 8 == 0 && !((uintptr_t)s.ptr % grid == 0 && (s.stride * 2) % grid == 0);
  };
  for (int i = 0; i < n; ++i)
    if (off(w[i], 128)) return phase512(w[i]);
  // (rows on the 128-byte grid reach here only from skip_sc1, which depends on
  // the row count; in batch-invariant mode they keep the aligned kernel's
  // lane mapping)
  if (batch_invariant()) return none;
  for (int i = 0; i < n; ++i)
    if (off(w[i], 512)) return phase512(w[i]);
  return none;
}

// The variant of a table entry for rows needs_unaligned() reports (or for
// calls skip_sc1() takes off the sc1 bits).  The variants of modes 0, 1, 3
// and 4 rotate their rows onto whole lines and keep the entry's sc1 bits for
// calls past 16 Mi elements: with 4096 rows 16 bytes off the grid (stride
// H + 8), sc1 and the 512-byte rotation measured 1.1-2.6% faster than
// neither at 12K-32K.  The tail variants keep them only past 2048 whole
// vectors (the 1024-lane rows: 1.1% faster at H = 32775; the LDS tier's tail
// variant at 16K measured 0.3-0.9% slower with them).  Smaller calls, and the
// FP8 and MX variants, which write partial lines (13-24% slower with sc1 at
// 16K-32K), go without.
int unaligned_flags(const Problem& p, int flags) {
  const bool tail = p.hidden % 8 != 0 || !(shift_phase(p) == Phase{0, 0});
  const bool rotated = p.mode == 0 || p.mode == 1 || p.mode == 3 || p.mode == 4;
  const bool keep_sc1 = rotated && p.rows * p.hidden > (int64_t(1) << 24) && (!tail || p.hidden / 8 > 2048);
  const int f = keep_sc1 ? flags : flags & ~24;
  return tail ? f | 96 : f | 32;
}

// The tail variants at exactly 2048 whole vectors take 1024 x 2 rather than
// the LDS tier's 256 x 8, whose edge registers (135 VGPRs) leave room for
// three workgroups per CU: 4096 rows of 16384 two bytes off the grid and of
// 16391, 4.4-5.1% faster in bf16 and fp16 (the unaligned variant, without
// the tail, keeps the LDS tier: within 0.5%).  The tail variants of 1024 x 2
// and 1024 x 3 load the weight late in every mode.
//
// A shifted row reads its weight 2-14 bytes off the weight's 16-byte vectors;
// from 1024 rows (plain RMSNorm: 384) the tail variants of 512 x 2-4 and
// 1024 x 2-3 instead stage the whole weight in LDS with aligned loads, once
// per workgroup (flags bit 14), where the fused op, its out-of-place and
// partial-sum forms measured 1.5-5% faster and plain RMSNorm 8-17% (4096
// rows, odd widths and rows two bytes off at 8K-20K).  Not below: the
// staging sits on a single row's critical path (1-256 rows: 3-23% slower);
// not in 1024 x 4 (1.7-3.5% slower: one workgroup per CU either way, VGPRs
// 80 -> 96), in the fused op's 1024 x 3 (62 -> 66 VGPRs: one workgroup per
// CU instead of two, -1.5% to +1.7%), nor the partial sums' 1024 x 2 (spills).
// (row counts on 256 CUs, as in table_config)
bool weight_in_lds(const Problem& p, int cus, const hprms_config& c) {
  if (c.lds_vec_per_lane != 0 || c.block_threads != c.lanes_per_row) return false;
  const int l = c.lanes_per_row, v = c.vec_per_lane;
  const int64_t r = rows_at_ref(p.rows, cus);
  switch (p.mode) {
    case 0:
    case 3: return r >= 1024 && ((l == 512 && (v == 2 || v == 3)) || (l == 1024 && v == 2));
    case 4: return r >= 1024 && l == 512 && v == 3;
    case 1: return r >= 384 && ((l == 512 && v >= 2 && v <= 4) || (l == 1024 && v == 3));
    default: return false;
  }
}

void tail_shape(const Problem& p, int cus, hprms_config* c) {
  if (!(c->flags & 64)) return;
  if (c->tier == 2 && c->lanes_per_row == 256)
    *c = hprms_config{1, 1024, 2, 0, 1024, c->grid_blocks, unaligned_flags(p, 31)};
  else if (c->lanes_per_row == 1024 && (c->vec_per_lane == 2 || c->vec_per_lane == 3))
    c->flags |= 4;
  if (weight_in_lds(p, cus, *c)) c->flags |= 16384;
}

// Calls that update the residual in place and whose input and residual rows
// fit in 64 MiB (rows x hidden <= 16 Mi elements) take the table's kernel
// without the sc1 bits: sc1 sends the stores past the 256 MB Infinity Cache.
// Measured at 512-2048 rows, H = 9216-32768, rows resident in the cache or
// not: the fused op 1-31% faster (9216 x 512 resident: 9.16 -> 6.36 us), the
// FP8 and MX outputs and the partial sums up to 9.5% (within +2.5% in the
// worst case).  Plain RMSNorm (+3-37%) and the out-of-place form (up to +13%
// with resident rows), whose inputs sc1 keeps in the cache, keep it.  Such
// calls run the shape's unaligned variant (flags bit 5, sc1 bits cleared; the
// registry has no aligned kernel of the shape without sc1): for rows on a
// 512-byte boundary it is the table kernel's mapping; rows on the 128-byte
// grid but off a 512-byte boundary are rotated onto one (rot_phase), which
// changes the order of the row's sum of squares, within the same bar (not in
// batch-invariant mode, where they keep the table kernel's mapping).
bool skip_sc1(const Problem& p) {
  return p.mode != 1 && p.mode != 3 && p.rows * p.hidden <= (int64_t(1) << 24);
}

// The general tier (hprms_general.hip): rows up to 16K elements stay in
// registers (one read and one write per element); longer rows take the
// two-pass kernel, which re-reads the residual row it has just written.
int launch_general(const Problem& p, hipStream_t stream) {
  GeneralArgs a = {};
  a.x = (const uint16_t*)p.x;
  a.out = (uint16_t*)(p.mode == 0 || p.mode == 2 ? p.x : p.out);
  a.res = (uint16_t*)p.res;
  a.w = (const uint16_t*)p.w;
  a.rows = p.rows;
  a.x_stride = p.x_stride;
  a.out_stride = p.mode == 0 || p.mode == 2 ? p.x_stride : p.out_stride;
  a.res_stride = p.res_stride;
  a.res_out = (uint16_t*)p.res_out;
  a.res_out_stride = p.res_out_stride;
  a.nparts = p.nparts;
  for (int g = 0; g < p.nparts && p.parts; ++g) a.parts[g] = (const uint16_t*)p.parts[g];
  a.hidden = p.hidden;
  a.hidden_f = (float)p.hidden;
  a.eps = (float)p.eps;
  a.q = p.mode == 2 ? (uint8_t*)p.out : nullptr;
  a.scale = p.scale;
  a.static_scale = p.static_scale;
  a.scale_ub = p.scale_ub;
  a.q_stride = p.mode == 2 ? p.out_stride : 0;
  const int64_t grid = p.rows < kMaxGrid ? p.rows : kMaxGrid;
  launch_general_kernels(a, p.dtype, p.mode, grid, stream);
  return check_launch("general rmsnorm kernel");
}

// Validates, picks the configuration and the kernel, then launches.  With
// rows == 0 everything but the launch still runs (pointers may be null), so a
// caller can check that a configuration exists without a device.
int run(const Problem& p, const hprms_config* forced, hipStream_t stream) {
  int rc = check_problem(p);
  if (rc != HPRMS_OK) return rc;

  hprms_config c;
  if (forced && forced->tier != 0) {
    c = *forced;
  } else {
    // (a call with no rows runs no kernel and asks no device)
    const int cus = p.rows > 0 ? current_cus() : kRefCUs;
    const bool off_grid = needs_unaligned(p);
    table_config(p.rows, p.hidden, p.mode, !off_grid, cus, &c);
    if (c.tier != 3 && (off_grid || ((c.flags & 24) && skip_sc1(p)))) {
      c.flags = unaligned_flags(p, c.flags);
      tail_shape(p, cus, &c);
    } else if (!off_grid && p.x_stride == p.res_stride) {
      // mode 7's scales in columns: one float per row, each group a column
      const bool scale_columns = p.mode == 7 && p.mx_scale_stride == 4 && p.hidden > 128;
      c.flags |= xcd_runs_flags(p.mode, p.rows, p.x_stride * 2, cus, c, scale_columns);
    }
  }
  if ((c.flags & 512) && !p.timeline)
    return fail(HPRMS_E_INVALID, "flags bit 9 (timeline) needs hprms_bench_fused_timeline and its buffer");
  if (is_blockq(p.mode) && (c.tier == 3 || !vec_fits(p, c)))
    return fail(HPRMS_E_INVALID,
                "%s output needs 2-byte aligned input, residual and weight, input and residual row "
                "strides below 2^31 elements and a row group's rows (strides times rows per "
                "workgroup) within 2 GiB", is_mx(p.mode) ? "MX" : "group-scaled FP8");
  if (c.tier != 3 && !vec_fits(p, c)) {
    if (forced && forced->tier != 0)
      return fail(HPRMS_E_INVALID,
                  "configuration (lanes_per_row %d, vec_per_lane %d) does not fit hidden %lld with "
                  "this alignment/stride", c.lanes_per_row, c.vec_per_lane, (long long)p.hidden);
    c.tier = 3;
  }
  if (c.tier == 3) {
    if (p.rows == 0) return HPRMS_OK;
    return launch_general(p, stream);
  }

  const FusedEntry* e = find_fused(p.dtype, p.mode, c);
  if (!e)
    return fail(HPRMS_E_INVALID,
                "no kernel built for (lanes_per_row %d, vec_per_lane %d, lds_vec_per_lane %d, "
                "block_threads %d, flags %d)", c.lanes_per_row, c.vec_per_lane, c.lds_vec_per_lane,
                c.block_threads, c.flags);
  if (p.rows == 0) return HPRMS_OK;

  // the kernel's leading scalar arguments (preloaded into SGPRs), then FusedArgs
  const uint16_t* x_rows = (const uint16_t*)p.x;
  // plain RMSNorm has no residual: the output takes its place
  uint16_t* res_rows = (uint16_t*)(p.mode == 1 ? p.out : p.res);
  const int64_t res_stride = p.mode == 1 ? p.out_stride : p.res_stride;
  const uint16_t* weight = (const uint16_t*)p.w;
  const int64_t rpb = c.block_threads / c.lanes_per_row;
  FusedArgs a = {};
  const int64_t ngroups = (p.rows + rpb - 1) / rpb;
  a.out = (uint16_t*)(p.mode == 0 || p.mode == 2 || is_blockq(p.mode) ? p.x : p.out);
  a.res_out = (uint16_t*)p.res_out;
  a.res_out_stride = p.res_out_stride;
  a.nparts = p.nparts;
  for (int g = 0; g < p.nparts && p.parts; ++g) a.parts[g] = (const uint16_t*)p.parts[g];
  a.q = p.mode == 2 || is_blockq(p.mode) ? (uint8_t*)p.out : nullptr;
  a.scale = p.scale;
  a.static_scale = p.static_scale;
  a.scale_ub = p.scale_ub;
  a.q_stride = p.mode == 2 || is_blockq(p.mode) ? p.out_stride : 0;
  a.mx_scale = (uint8_t*)p.mx_scales;
  a.mx_scale_stride = p.mx_scale_stride;
  a.mx_group_stride = p.mx_group_stride;
  a.out_stride = p.mode == 0 || p.mode == 2 || is_blockq(p.mode) ? p.x_stride : p.out_stride;
  const Phase shift = (c.flags & 64) ? shift_phase(p) : Phase{0, 0};
  const Phase rot = (c.flags & 32) ? rot_phase(p) : Phase{0, 0};
  const uint32_t phases = pack_phases(rot.base, rot.step, shift.base, shift.step);
  a.timeline = p.timeline;

  int64_t grid = ngroups;
  if (c.grid_blocks > 0 && c.grid_blocks < grid) grid = c.grid_blocks;
  if (grid > kMaxGrid) grid = kMaxGrid;
  // flags bit 11: 96 KiB of (unused) dynamic LDS, so one workgroup holds a CU
  const unsigned lds = (c.flags & 2048) ? 96u * 1024u : 0u;
  hipLaunchKernelGGL(e->fn, dim3((unsigned)grid), dim3(c.block_threads), lds, stream, x_rows, res_rows, weight,
                     p.rows, (int32_t)p.x_stride, (int32_t)res_stride, (int32_t)p.hidden, (int32_t)grid, phases,
                     (float)p.eps, a);
  return check_launch("fused rmsnorm kernel");
}

// ---- streamer ---------------------------------------------------------------------
template <int DT, int OP>
int launch_stream(const StreamArgs& base, bool flat, hipStream_t stream) {
  StreamArgs a = base;
  if (flat) {
    // One 16-byte vector per lane, 256 lanes (4 KiB) per workgroup: short-lived
    // workgroups over a contiguous window measured fastest on gfx950
    // (6.3 TB/s for a 235 MB copy, against 5.2 TB/s for a persistent grid).
    constexpr int kBlock = 256, kUnroll = 1;
    a.nvec = (a.rows * a.hidden) / 8;
    int64_t grid = (a.nvec + (int64_t)kBlock * kUnroll - 1) / ((int64_t)kBlock * kUnroll);
    if (grid < 1) grid = 1;
    if (grid > kMaxGrid)
      return fail(HPRMS_E_RANGE, "streamer: %lld elements exceed the grid limit", (long long)(a.rows * a.hidden));
    stream_chunk_kernel<DT, OP, kUnroll, kBlock><<<dim3((unsigned)grid), dim3(kBlock), 0, stream>>>(a.in, a.out,
                                                                                                 a.nvec, a);
  } else {
    // strided or misaligned rows: 4 KiB chunks of a row per workgroup
    constexpr int kBlock = 256;
    a.nvec = a.hidden / 8;
    const int64_t chunks = a.nvec > 0 ? (a.nvec + kBlock - 1) / kBlock : 1;
    const int64_t units = a.rows * chunks;
    const int64_t grid = units < kMaxGrid ? units : kMaxGrid;
    stream_rows_kernel<DT, OP, kBlock><<<dim3((unsigned)grid), dim3(kBlock), 0, stream>>>(
        a.in, a.out, a.rows, a.in_stride, a.out_stride, (int32_t)a.hidden, (int32_t)a.nvec, (int32_t)grid);
  }
  return check_launch("streamer kernel");
}

}  // namespace
}  // namespace hprms

using namespace hprms;

extern "C" {

int hprms_fused_add_rmsnorm(void* input, const void* weight, void* residual, int64_t rows, int64_t hidden,
                            int64_t input_row_stride, int64_t residual_row_stride, int dtype, double eps,
                            hipStream_t stream) {
  Problem p{0, input, input, residual, weight, rows, hidden, input_row_stride, input_row_stride,
            residual_row_stride, dtype, eps, nullptr};
  return run(p, nullptr, stream);
}

int hprms_fused_add_rmsnorm_fp8(void* out, float* scale, const void* input, const void* weight, void* residual,
                                int64_t rows, int64_t hidden, int64_t out_row_stride, int64_t input_row_stride,
                                int64_t residual_row_stride, int dtype, double eps, hipStream_t stream) {
  Problem p{2, const_cast<void*>(input), out, residual, weight, rows, hidden, input_row_stride, out_row_stride,
            residual_row_stride, dtype, eps, scale};
  return run(p, nullptr, stream);
}

int hprms_fused_add_rmsnorm_fp8_ub(void* out, float* scale, const float* scale_ub, const void* input,
                                   const void* weight, void* residual, int64_t rows, int64_t hidden,
                                   int64_t out_row_stride, int64_t input_row_stride, int64_t residual_row_stride,
                                   int dtype, double eps, hipStream_t stream) {
  Problem p{2, const_cast<void*>(input), out, residual, weight, rows, hidden, input_row_stride, out_row_stride,
            residual_row_stride, dtype, eps, scale};
  p.scale_ub = scale_ub;
  if (!scale_ub && rows > 0) return fail(HPRMS_E_INVALID, "null tensor pointer (scale_ub)");
  return run(p, nullptr, stream);
}

int hprms_fused_add_rmsnorm_fp8_static(void* out, const float* scale, const void* input, const void* weight,
                                       void* residual, int64_t rows, int64_t hidden, int64_t out_row_stride,
                                       int64_t input_row_stride, int64_t residual_row_stride, int dtype, double eps,
                                       hipStream_t stream) {
  Problem p{2, const_cast<void*>(input), out, residual, weight, rows, hidden, input_row_stride, out_row_stride,
            residual_row_stride, dtype, eps, nullptr};
  p.static_scale = scale;
  return run(p, nullptr, stream);
}

int hprms_fused_add_rmsnorm_config(void* input, const void* weight, void* residual, int64_t rows,
                                   int64_t hidden, int64_t input_row_stride, int64_t residual_row_stride,
                                   int dtype, double eps, const hprms_config* config, hipStream_t stream) {
  if (!config) return fail(HPRMS_E_INVALID, "config is null");
  Problem p{0, input, input, residual, weight, rows, hidden, input_row_stride, input_row_stride,
            residual_row_stride, dtype, eps, nullptr};
  return run(p, config, stream);
}

int hprms_fused_add_rmsnorm_out(void* out, void* residual_out, const void* input, const void* residual,
                                const void* weight, int64_t rows, int64_t hidden, int64_t out_row_stride,
                                int64_t residual_out_row_stride, int64_t input_row_stride,
                                int64_t residual_row_stride, int dtype, double eps, hipStream_t stream) {
  Problem p{3, const_cast<void*>(input), out, const_cast<void*>(residual), weight, rows, hidden, input_row_stride,
            out_row_stride, residual_row_stride, dtype, eps};
  p.res_out = residual_out;
  p.res_out_stride = residual_out_row_stride;
  return run(p, nullptr, stream);
}

int hprms_reduce_add_rmsnorm(void* out, const void* const* parts, int nparts, const void* weight, void* residual,
                             int64_t rows, int64_t hidden, int64_t out_row_stride, int64_t part_row_stride,
                             int64_t residual_row_stride, int dtype, double eps, hipStream_t stream) {
  Problem p{4, nullptr, out, residual, weight, rows, hidden, part_row_stride, out_row_stride,
            residual_row_stride, dtype, eps};
  p.nparts = nparts;
  p.parts = parts;
  if (parts && nparts >= 1) p.x = const_cast<void*>(parts[0]);
  return run(p, nullptr, stream);
}

int hprms_fused_add_rmsnorm_mx(void* out, void* scales, const void* input, const void* weight, void* residual,
                               int64_t rows, int64_t hidden, int64_t out_row_stride, int64_t scale_row_stride,
                               int64_t input_row_stride, int64_t residual_row_stride, int format, int dtype,
                               double eps, hipStream_t stream) {
  if (format != HPRMS_MX_FP8_E4M3 && format != HPRMS_MX_FP4_E2M1)
    return fail(HPRMS_E_INVALID, "format must be HPRMS_MX_FP8_E4M3 or HPRMS_MX_FP4_E2M1 (got %d)", format);
  Problem p{format == HPRMS_MX_FP8_E4M3 ? 5 : 6, const_cast<void*>(input), out, residual, weight, rows, hidden,
            input_row_stride, out_row_stride, residual_row_stride, dtype, eps};
  p.mx_scales = scales;
  p.mx_scale_stride = scale_row_stride;
  return run(p, nullptr, stream);
}

int hprms_fused_add_rmsnorm_fp8_group(void* out, float* scales, const void* input, const void* weight,
                                      void* residual, int64_t rows, int64_t hidden, int64_t out_row_stride,
                                      int64_t scale_row_stride, int64_t scale_group_stride,
                                      int64_t input_row_stride, int64_t residual_row_stride, int dtype, double eps,
                                      hipStream_t stream) {
  // the kernels take the scale strides in bytes
  if (scale_row_stride < 0 || scale_row_stride > (int64_t(1) << 40) || scale_group_stride < 0 ||
      scale_group_stride > (int64_t(1) << 40))
    return fail(HPRMS_E_INVALID, "scale strides (row %lld, group %lld) out of range [0, 2^40]",
                (long long)scale_row_stride, (long long)scale_group_stride);
  Problem p{7, const_cast<void*>(input), out, residual, weight, rows, hidden, input_row_stride, out_row_stride,
            residual_row_stride, dtype, eps};
  p.mx_scales = scales;
  p.mx_scale_stride = scale_row_stride * 4;
  p.mx_group_stride = scale_group_stride * 4;
  return run(p, nullptr, stream);
}

int hprms_rmsnorm(void* out, const void* in, const void* weight, int64_t rows, int64_t hidden,
                  int64_t out_row_stride, int64_t in_row_stride, int dtype, double eps, hipStream_t stream) {
  Problem p{1, const_cast<void*>(in), out, nullptr, weight, rows, hidden, in_row_stride, out_row_stride,
            0, dtype, eps, nullptr};
  return run(p, nullptr, stream);
}

int hprms_select_config_cu(int64_t rows, int64_t hidden, int dtype, int mode, int cu_count,
                           hprms_config* config) {
  if (!config) return fail(HPRMS_E_INVALID, "config is null");
  if (dtype != HPRMS_DTYPE_BF16 && dtype != HPRMS_DTYPE_FP16)
    return fail(HPRMS_E_INVALID, "dtype must be HPRMS_DTYPE_BF16 or HPRMS_DTYPE_FP16 (got %d)", dtype);
  if (mode < 0 || mode > 7) return fail(HPRMS_E_INVALID, "mode must be in [0, 7] (got %d)", mode);
  if (rows < 0 || hidden < 1 || hidden > kMaxHidden) return fail(HPRMS_E_INVALID, "bad rows/hidden");
  if (cu_count < 1 || cu_count > 65536) return fail(HPRMS_E_INVALID, "cu_count must be in [1, 65536] (got %d)", cu_count);
  // the choice for rows on the 128-byte grid; odd widths: the tail variant of
  // the choice for rows off it
  table_config(rows, hidden, mode, hidden % 8 == 0, cu_count, config);
  if (hidden % 8 == 0) config->flags |= xcd_runs_flags(mode, rows, hidden * 2, cu_count, *config, false);
  if (hidden % 8 != 0) {
    if (config->tier != 3 && hidden >= 8 && mode <= 4) {
      Problem p{mode, nullptr, nullptr, nullptr, nullptr, rows, hidden, hidden, hidden, hidden, dtype, 0.0};
      config->flags = unaligned_flags(p, config->flags);
      tail_shape(p, cu_count, config);
    } else {
      config->tier = 3;
    }
  }
  return HPRMS_OK;
}

int hprms_set_batch_invariant(int enable) {
  if (enable != 0 && enable != 1) return fail(HPRMS_E_INVALID, "enable must be 0 or 1 (got %d)", enable);
  const int previous = hprms::batch_invariant() ? 1 : 0;
  hprms::g_batch_invariant.store(enable, std::memory_order_relaxed);
  return previous;
}

int hprms_batch_invariant(void) { return hprms::batch_invariant() ? 1 : 0; }

int hprms_select_config(int64_t rows, int64_t hidden, int dtype, int mode, hprms_config* config) {
  return hprms_select_config_cu(rows, hidden, dtype, mode, kRefCUs, config);
}

int hprms_device_cu_count(int device) {
  if (device < 0) {
    if (hipGetDevice(&device) != hipSuccess) {
      const hipError_t e = hipGetLastError();
      return fail(HPRMS_E_LAUNCH, "no current device: %s", hipGetErrorString(e));
    }
  }
  return device_cus(device);
}

int hprms_streamer(void* out, const void* in, int64_t rows, int64_t hidden, int64_t out_row_stride,
                   int64_t in_row_stride, int dtype, int op, hipStream_t stream) {
  if (dtype != HPRMS_DTYPE_BF16 && dtype != HPRMS_DTYPE_FP16)
    return fail(HPRMS_E_INVALID, "dtype must be HPRMS_DTYPE_BF16 or HPRMS_DTYPE_FP16 (got %d)", dtype);
  if (op != HPRMS_STREAM_COPY && op != HPRMS_STREAM_RELU)
    return fail(HPRMS_E_INVALID, "op must be HPRMS_STREAM_COPY or HPRMS_STREAM_RELU (got %d)", op);
  if (rows < 0) return fail(HPRMS_E_INVALID, "rows must be >= 0 (got %lld)", (long long)rows);
  if (hidden < 1) return fail(HPRMS_E_INVALID, "hidden must be >= 1 (got %lld)", (long long)hidden);
  if (out_row_stride < hidden || in_row_stride < hidden)
    return fail(HPRMS_E_INVALID, "row strides must be >= hidden");
  if (hidden >= (int64_t(1) << 30))  // a row's buffer resource spans 2 * hidden < 2^31 bytes
    return fail(HPRMS_E_RANGE, "hidden %lld exceeds the streamer's row limit 2^30 - 1", (long long)hidden);
  if (rows == 0) return HPRMS_OK;
  if (!extent_ok(rows, out_row_stride, 2, hidden) || !extent_ok(rows, in_row_stride, 2, hidden))
    return fail(HPRMS_E_RANGE, "%lld rows at these row strides span more than 2^56 bytes", (long long)rows);
  if (!out || !in) return fail(HPRMS_E_INVALID, "null tensor pointer");
  StreamArgs a{(uint16_t*)out, (const uint16_t*)in, rows, hidden, out_row_stride, in_row_stride, 0};
  const bool flat = out_row_stride == hidden && in_row_stride == hidden && aligned16(out) && aligned16(in);
  if (dtype == HPRMS_DTYPE_BF16)
    return op == HPRMS_STREAM_COPY ? launch_stream<HPRMS_DTYPE_BF16, HPRMS_STREAM_COPY>(a, flat, stream)
                                   : launch_stream<HPRMS_DTYPE_BF16, HPRMS_STREAM_RELU>(a, flat, stream);
  return op == HPRMS_STREAM_COPY ? launch_stream<HPRMS_DTYPE_FP16, HPRMS_STREAM_COPY>(a, flat, stream)
                                 : launch_stream<HPRMS_DTYPE_FP16, HPRMS_STREAM_RELU>(a, flat, stream);
}

int hprms_kernel_configs(int dtype, int mode, hprms_config* out, int capacity) {
  if (dtype != HPRMS_DTYPE_BF16 && dtype != HPRMS_DTYPE_FP16)
    return fail(HPRMS_E_INVALID, "dtype must be HPRMS_DTYPE_BF16 or HPRMS_DTYPE_FP16 (got %d)", dtype);
  if (mode < 0 || mode > 7) return fail(HPRMS_E_INVALID, "mode must be in [0, 7] (got %d)", mode);
  if (capacity < 0 || (capacity > 0 && !out)) return fail(HPRMS_E_INVALID, "bad output array");
  int n = 0;
  for (const Registry& r : kRegistries) {
    for (int i = 0; i < r.count; ++i) {
      const FusedEntry& e = r.entries[i];
      if (e.dtype != dtype || e.mode != mode) continue;
      const hprms_config c{e.ldsv > 0 ? 2 : 1, e.lpr, e.vpl, e.ldsv, e.block, 0, e.flags};
      if (find_fused(dtype, mode, c) != &e) continue;  // listed once: the lookup's first match
      if (n < capacity) out[n] = c;
      ++n;
    }
  }
  return n;
}

#ifdef HPRMS_BENCH_BUILD
// Bench library only: the in-place fused op on contiguous rows with a forced
// configuration whose flags carry bit 9, recording per workgroup {start, end,
// HW_ID, XCC_ID} (realtime clock ticks of 10 ns) into timeline[4 * workgroup
// + i]; the caller sizes timeline for the launched grid.
int hprms_bench_fused_timeline(void* input, const void* weight, void* residual, int64_t rows, int64_t hidden,
                               int dtype, double eps, const hprms_config* config, int64_t* timeline,
                               hipStream_t stream) {
  if (!config) return fail(HPRMS_E_INVALID, "config is null");
  Problem p{0, input, input, residual, weight, rows, hidden, hidden, hidden, hidden, dtype, eps, nullptr};
  p.timeline = timeline;
  return run(p, config, stream);
}

// Bench library only: one of the fused op's other forms on contiguous rows
// with a forced configuration, to time the table's shape against its
// variants (the row-group order).  mode 1: `out` <- plain RMSNorm of `input`
// (no residual); 3: `out` and `aux` (the residual output) out of place; 2:
// FP8 with per-row scales in `aux`; 5 / 6: MXFP8 / MXFP4, hidden / 32 scale
// bytes per row in `aux`; 7: float32 scales per 128 elements in `aux` at
// (aux_row_stride, aux_group_stride) elements.
int hprms_bench_form_config(int mode, void* out, void* aux, int64_t aux_row_stride, int64_t aux_group_stride,
                            void* input, const void* weight, void* residual, int64_t rows, int64_t hidden,
                            int dtype, double eps, const hprms_config* config, hipStream_t stream) {
  if (!config) return fail(HPRMS_E_INVALID, "config is null");
  if (mode != 1 && mode != 2 && mode != 3 && mode != 5 && mode != 6 && mode != 7)
    return fail(HPRMS_E_INVALID, "mode must be 1, 2, 3, 5, 6 or 7 (got %d)", mode);
  if (aux_row_stride < 0 || aux_row_stride > (int64_t(1) << 40) || aux_group_stride < 0 ||
      aux_group_stride > (int64_t(1) << 40))
    return fail(HPRMS_E_INVALID, "scale strides out of range [0, 2^40]");
  const bool quant = mode == 2 || mode >= 5;
  Problem p{mode, input, out, mode == 1 ? nullptr : residual, weight, rows, hidden, hidden,
            quant ? q_row_bytes(mode, hidden) : hidden, mode == 1 ? 0 : hidden, dtype, eps, nullptr};
  if (mode == 2) {
    p.scale = (float*)aux;
  } else if (mode == 3) {
    p.res_out = aux;
    p.res_out_stride = hidden;
  } else if (mode >= 5) {
    p.mx_scales = aux;
    p.mx_scale_stride = mode == 7 ? aux_row_stride * 4 : aux_row_stride;
    p.mx_group_stride = aux_group_stride * 4;
  }
  return run(p, config, stream);
}
#endif

const char* hprms_last_error(void) { return g_err; }

int hprms_abi_version(void) { return HPRMS_ABI_VERSION; }

}  // extern "C"
