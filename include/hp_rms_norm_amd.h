/*
 * hp_rms_norm_amd.h - C ABI of the MI355X (gfx950) fused residual-add + RMSNorm
 * library `libhprms.so`.
 *
 * Every entry point takes plain device pointers, element counts, element
 * strides, a dtype code and a HIP stream.  No entry point allocates device
 * memory, synchronises the stream or throws: each returns HPRMS_OK (0) or a
 * negative HPRMS_E* code, and the message of the calling thread's last failure
 * is available from hprms_last_error().  Launches are asynchronous on `stream`
 * (NULL = the null stream of the current device).  The kernels run on the
 * device that owns the pointers; the caller makes that device current.
 *
 * Storage is row-major [rows, hidden] with a row stride (in elements) per
 * tensor; elements inside a row are contiguous.
 */
#ifndef HP_RMS_NORM_AMD_H_
#define HP_RMS_NORM_AMD_H_

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HPRMS_ABI_VERSION 8

/* element types (the reference accepts exactly these two:
 * hp_rms_norm/csrc/cuda/hp_rms_norm.cu:29-49) */
typedef enum {
  HPRMS_DTYPE_BF16 = 0,
  HPRMS_DTYPE_FP16 = 1
} hprms_dtype;

/* status codes */
#define HPRMS_OK 0
#define HPRMS_E_INVALID (-22)  /* bad argument: null pointer, size, stride, dtype */
#define HPRMS_E_LAUNCH (-5)    /* the HIP runtime rejected a launch or query */
#define HPRMS_E_RANGE (-34)    /* a size or stride does not fit the kernel's index width, or a
                                  tensor's rows span more than 2^56 bytes */

/* most partial buffers hprms_reduce_add_rmsnorm() sums */
#define HPRMS_MAX_PARTS 8

/* element formats of hprms_fused_add_rmsnorm_mx() (OCP Microscaling Formats v1.0) */
#define HPRMS_MX_FP8_E4M3 0   /* MXFP8: one E4M3 byte per element */
#define HPRMS_MX_FP4_E2M1 1   /* MXFP4: two E2M1 codes per byte, the even element in the low nibble */

/* streamer operations for hprms_streamer() */
#define HPRMS_STREAM_COPY 0   /* out = in (the reference "relu": activation_kernels.cuh:99-119) */
#define HPRMS_STREAM_RELU 1   /* out = max(in, +0), NaN propagates */

/*
 * Fused residual-add + RMSNorm, in place.
 *   residual[r, :] <- rne(f32(input) + f32(residual))
 *   input[r, :]    <- rne((f32(residual_new) * rsqrt(mean(f32(residual_new)^2) + eps)) * f32(weight))
 * with fp32 accumulation of the mean of squares.
 *
 * Replaces the reference's host entry `void rms_norm(Tensor& input, const
 * Tensor& weight, Tensor& residual, double eps)` (hp_rms_norm/csrc/cuda/hp_rms_norm.cu:7-50)
 * and its launcher `launch_rms_norm<T>(T* input, const T* weight, T* residual,
 * size_t tokens, int hidden_dim, double eps, cudaStream_t)`
 * (hp_rms_norm/csrc/cuda/hp_rms_norm.cuh:562-618); the two row strides are new
 * (the reference assumes contiguous rows).  rows == 0 is a no-op.
 * hidden may be any value in [1, 2^24] and rows may start at any 2-byte
 * boundary.  The vector tiers take every hidden in [8, 65543]: rows off the
 * 128-byte grid run a variant that rotates each row's lane mapping onto
 * 512-byte boundaries of the input (whole cache lines), hidden % 8 != 0 adds
 * a tail vector, and from hidden 4104 up, when neither input nor residual has
 * its rows on 16-byte boundaries, the rows are shifted so that the input is
 * accessed aligned (flags bits 5 and 6 of hprms_config); other shapes take a
 * slower general kernel.  The results
 * meet the same bar in every case: residual bit-exact, output within 1 ulp
 * of the reference formula.
 */
int hprms_fused_add_rmsnorm(void* input, const void* weight, void* residual,
                            int64_t rows, int64_t hidden,
                            int64_t input_row_stride, int64_t residual_row_stride,
                            int dtype, double eps, hipStream_t stream);

/*
 * Row-wise streamer: out[r, :] = op(in[r, :]).
 * Replaces `void relu(Tensor& out, const Tensor& input)`
 * (hp_rms_norm/csrc/cuda/activation_kernels.cu:7-39) and `launch_relu<T>(const T*
 * input, T* out, int64_t tokens, int dim, int sm_count, cudaStream_t)`
 * (hp_rms_norm/csrc/cuda/activation_kernels.cuh:122-145).  HPRMS_STREAM_COPY
 * is the reference's observable behaviour (an identity copy); HPRMS_STREAM_RELU
 * is a true ReLU offered beside it.  `out` and `in` must not partially overlap.
 */
int hprms_streamer(void* out, const void* in, int64_t rows, int64_t hidden,
                   int64_t out_row_stride, int64_t in_row_stride,
                   int dtype, int op, hipStream_t stream);

/*
 * Plain (residual-free) RMSNorm, out of place: out = rne((f32(in) * rsqrt(mean(f32(in)^2) + eps)) * f32(weight)).
 * No counterpart in the reference; it is the same kernel family without the
 * residual stream, for the first and last norm of a layer stack.
 * `out` may equal `in` (in place).
 */
int hprms_rmsnorm(void* out, const void* in, const void* weight,
                  int64_t rows, int64_t hidden,
                  int64_t out_row_stride, int64_t in_row_stride,
                  int dtype, double eps, hipStream_t stream);

/*
 * Fused residual-add + RMSNorm with an FP8 (OCP e4m3fn) output and one scale
 * per row (dynamic per-token quantisation of the op's 16-bit output y):
 *   residual[r, :] <- rne16(f32(input) + f32(residual))        (in place)
 *   y              =  the 16-bit output of hprms_fused_add_rmsnorm
 *   scale[r]       =  max(max_j |y[r, j]| / 448, FLT_MIN)      (float32)
 *   out[r, :]      =  e4m3fn(clamp(y / scale[r] computed as y * (1 / scale[r]), -448, 448))
 * `input` is only read; `out` is [rows, hidden] bytes with its own row stride
 * (in bytes).  A row containing NaN gets a NaN scale and NaN outputs.  No
 * counterpart in the reference: it is the fused op followed by the
 * quantisation step that feeds an FP8 GEMM, with one write of H bytes
 * instead of 2H.  `out` may start at any byte.
 */
int hprms_fused_add_rmsnorm_fp8(void* out, float* scale, const void* input, const void* weight,
                                void* residual, int64_t rows, int64_t hidden, int64_t out_row_stride,
                                int64_t input_row_stride, int64_t residual_row_stride,
                                int dtype, double eps, hipStream_t stream);

/*
 * hprms_fused_add_rmsnorm_fp8 with an upper bound on each row's maximum
 * (the activation scale bound of FP8 row-wise checkpoints):
 *   scale[r] = max(min(max_j |y[r, j]|, *scale_ub) / 448, FLT_MIN)
 * and out as above with that scale.  `scale_ub` is one float32 in device
 * memory, read by the kernel (so a captured graph sees later values); a row
 * containing NaN keeps a NaN scale, and a NaN bound bounds nothing.  No
 * counterpart in the reference.
 */
int hprms_fused_add_rmsnorm_fp8_ub(void* out, float* scale, const float* scale_ub, const void* input,
                                   const void* weight, void* residual, int64_t rows, int64_t hidden,
                                   int64_t out_row_stride, int64_t input_row_stride,
                                   int64_t residual_row_stride, int dtype, double eps, hipStream_t stream);

/*
 * The same with one scale for every row, given by the caller (static
 * per-tensor quantisation, the scale calibrated offline for the FP8 GEMM that
 * follows):
 *   out[r, :] = e4m3fn(clamp(y * (1 / scale[0]), -448, 448))
 * `scale` points to one float32 on the device and is only read (a scale of 0
 * gives +-448 and NaN for y = 0; a NaN scale gives NaN).  No row maximum is
 * taken and no scale is written.  No counterpart in the reference.
 */
int hprms_fused_add_rmsnorm_fp8_static(void* out, const float* scale, const void* input,
                                       const void* weight, void* residual, int64_t rows,
                                       int64_t hidden, int64_t out_row_stride,
                                       int64_t input_row_stride, int64_t residual_row_stride,
                                       int dtype, double eps, hipStream_t stream);

/*
 * Fused residual-add + RMSNorm out of place: the arithmetic of
 * hprms_fused_add_rmsnorm() with `input` and `residual` only read,
 *   residual_out[r, :] <- rne(f32(input) + f32(residual))
 *   out[r, :]          <- the normalised output
 * No counterpart in the reference (its op is in place only,
 * hp_rms_norm/csrc/cuda/hp_rms_norm.cu:33,42); it moves the same 4 rows of
 * bytes per row as the in-place op, where a clone followed by the in-place op
 * moves 8.  `out` may equal `input` and `residual_out` may equal `residual`
 * (exact aliases with equal strides, i.e. in place); `out` and
 * `residual_out` must differ.  Buffers must not otherwise overlap.
 */
int hprms_fused_add_rmsnorm_out(void* out, void* residual_out, const void* input, const void* residual,
                                const void* weight, int64_t rows, int64_t hidden,
                                int64_t out_row_stride, int64_t residual_out_row_stride,
                                int64_t input_row_stride, int64_t residual_row_stride,
                                int dtype, double eps, hipStream_t stream);

/*
 * Partial-sum reduction fused with residual-add + RMSNorm: the on-device half
 * of a tensor-parallel "all-reduce + residual + RMSNorm".  With P = nparts
 * (1 ... HPRMS_MAX_PARTS) buffers of the same shape and row stride,
 *   a[r, :]        =  rne(((f32(parts[0]) + f32(parts[1])) + ...) + f32(parts[P-1]))
 *   residual[r, :] <- rne(f32(a) + f32(residual))                 (in place)
 *   out[r, :]      <- rne((f32(residual_new) * rsqrt(mean(f32(residual_new)^2) + eps)) * f32(weight))
 * i.e. an all-reduce that sums in fp32 in rank order and rounds once, followed
 * by hprms_fused_add_rmsnorm() on its result; with P = 1 it equals that op
 * writing to `out`.  The parts are only read: in a deployment they are the
 * peer buffers of the ranks (device pointers mapped from the other GPUs) or
 * the chunks a reduce-scatter received.  No counterpart in the reference.
 * `out` may be one of the parts (exact alias, same row stride); `residual`
 * must not alias `out` or a part.
 */
int hprms_reduce_add_rmsnorm(void* out, const void* const* parts, int nparts, const void* weight,
                             void* residual, int64_t rows, int64_t hidden, int64_t out_row_stride,
                             int64_t part_row_stride, int64_t residual_row_stride,
                             int dtype, double eps, hipStream_t stream);

/*
 * Fused residual-add + RMSNorm with an OCP MX block-scaled output (the input
 * format of gfx950's scaled MFMA instructions):
 *   residual[r, :] <- rne16(f32(input) + f32(residual))        (in place)
 *   y              =  the 16-bit output of hprms_fused_add_rmsnorm
 *   per block of 32 consecutive elements of a row:
 *     s          = clamp(floor(log2(max |y|)) - emax, -127, 127)   (emax 8 for E4M3, 2 for E2M1)
 *     scales[b]  = s + 127 (E8M0; 0xFF if the block holds a NaN or an infinity)
 *     out        = y / 2^s rounded to nearest even in the element format,
 *                  saturated to +-448 (E4M3) or +-6 (E2M1)
 * `format` is HPRMS_MX_FP8_E4M3 (out: hidden bytes per row) or
 * HPRMS_MX_FP4_E2M1 (out: hidden / 2 bytes per row); `scales` holds hidden / 32
 * bytes per row; both row strides are in bytes.  `input` is only read.  Needs
 * hidden % 32 == 0, 2-byte aligned input, residual and weight (`out` and
 * `scales` may start at any byte), and input and residual row strides below
 * 2^31 elements; there is no general-tier fallback, so a row group (rows per
 * workgroup times the row strides) must also span < 2 GiB.  Other calls
 * return HPRMS_E_INVALID.
 * No counterpart in the reference.
 */
int hprms_fused_add_rmsnorm_mx(void* out, void* scales, const void* input, const void* weight,
                               void* residual, int64_t rows, int64_t hidden, int64_t out_row_stride,
                               int64_t scale_row_stride, int64_t input_row_stride,
                               int64_t residual_row_stride, int format, int dtype, double eps,
                               hipStream_t stream);

/*
 * Fused residual-add + RMSNorm with an FP8 (OCP e4m3fn) output and one
 * float32 scale per 128 consecutive elements of a row (per-token-group
 * quantisation, 1 x 128 groups, the activation format of block-scaled FP8
 * GEMMs):
 *   residual[r, :] <- rne16(f32(input) + f32(residual))        (in place)
 *   y              =  the 16-bit output of hprms_fused_add_rmsnorm
 *   per group g of 128 consecutive elements of row r:
 *     scales[r, g] =  max(max |y| / 448, FLT_MIN)   (NaN if the group holds a NaN)
 *     out          =  e4m3fn(clamp(y * (1 / scales[r, g]), -448, 448))
 * `out` is [rows, hidden] bytes with its row stride in bytes.  `scales` is
 * float32, 4-byte aligned; scales[r, g] sits at element
 * r * scale_row_stride + g * scale_group_stride: rows of scales
 * (scale_group_stride 1, scale_row_stride >= hidden / 128) or the
 * column-major, token-minor layout some block-scaled GEMMs read
 * (scale_row_stride 1, scale_group_stride >= rows, e.g. rows rounded up to a
 * multiple of 4).  Any strides in [0, 2^40] under which no two (row, group)
 * pairs share a scale are taken: the scales form rows (scale_row_stride >
 * (hidden / 128 - 1) * scale_group_stride, scale_group_stride >= 1) or
 * columns (scale_group_stride > (rows - 1) * scale_row_stride,
 * scale_row_stride >= 1).  `input` is only read.  Needs hidden % 128 == 0
 * and the same layouts as hprms_fused_add_rmsnorm_mx (no general-tier
 * fallback; a row group's scales, too, within 2 GiB); other calls return
 * HPRMS_E_INVALID.  No counterpart in the reference.
 */
int hprms_fused_add_rmsnorm_fp8_group(void* out, float* scales, const void* input, const void* weight,
                                      void* residual, int64_t rows, int64_t hidden,
                                      int64_t out_row_stride, int64_t scale_row_stride,
                                      int64_t scale_group_stride, int64_t input_row_stride,
                                      int64_t residual_row_stride, int dtype, double eps,
                                      hipStream_t stream);

/*
 * Kernel configuration of the fused add+RMSNorm family.  Used by the tuning
 * sweep and by tests that exercise every tier at every shape; normal callers
 * use hprms_fused_add_rmsnorm(), which picks the configuration from the
 * gfx950 table.  No counterpart in the reference (its tier choice is internal
 * to launch_rms_norm, hp_rms_norm.cuh:573).
 */
typedef struct {
  int32_t tier;             /* 0 = table, 1 = register tier, 2 = register+LDS tier, 3 = general kernel */
  int32_t lanes_per_row;    /* 16, 32, 64, 128, 256, 512 or 1024 */
  int32_t vec_per_lane;     /* 16-byte vectors of the row held by each lane */
  int32_t lds_vec_per_lane; /* of those, how many are kept in LDS (tier 2) */
  int32_t block_threads;    /* workgroup size: 64 ... 1024 */
  int32_t grid_blocks;      /* 0 = one workgroup per row group; >0 = persistent grid of this many */
  int32_t flags;            /* bit 0: non-temporal row loads; bit 1: non-temporal stores;
                               bit 2: weight loaded after the residual is stored;
                               bit 3 / bit 4: sc1 cache-policy bit on the row loads / stores;
                               bit 5: variant for rows off the 128-byte grid (any 2-byte
                               boundary; in modes 0, 1, 3, 4 each row's lane mapping rotated
                               so that every wave's access starts on a cache line of the
                               first written tensor), bit 6 (with bit 5): head and tail vectors, for
                               hidden % 8 != 0 and (from hidden 4104 up, modes 0-4) rows
                               shifted to the first written tensor's 16-byte phase;
                               bit 7: a lane's residual loads issued before its input loads;
                               bit 14 (with bit 6, late weight, rows of several waves, not
                               the FP8 output): the whole weight loaded once per workgroup
                               with aligned loads into LDS, where shifted rows read it;
                               bit 15 (partial sums, the latency rows): every part's loads
                               issued before the first part is added;
                               bits 16-18, V > 0 (the in-place op and the quantised
                               outputs at some row pitches): each XCD takes runs of 2^V
                               consecutive row groups rather than every 8th (the same
                               results) */
} hprms_config;

int hprms_fused_add_rmsnorm_config(void* input, const void* weight, void* residual,
                                   int64_t rows, int64_t hidden,
                                   int64_t input_row_stride, int64_t residual_row_stride,
                                   int dtype, double eps, const hprms_config* config,
                                   hipStream_t stream);

/* The configuration the library would use for (rows, hidden, dtype) and
 * `mode` (0: hprms_fused_add_rmsnorm, 1: hprms_rmsnorm, 2:
 * hprms_fused_add_rmsnorm_fp8, 3: hprms_fused_add_rmsnorm_out, 4:
 * hprms_reduce_add_rmsnorm, 5 / 6: hprms_fused_add_rmsnorm_mx with
 * HPRMS_MX_FP8_E4M3 / HPRMS_MX_FP4_E2M1, 7: hprms_fused_add_rmsnorm_fp8_group,
 * which takes the MX modes' shapes) on a device of 256 CUs (a whole
 * MI355X), written to *config; tier 3 when only the general kernel fits
 * hidden.  It is the choice for contiguous rows on the 128-byte grid (for
 * hidden % 8 != 0: the tail variant of the choice for rows off it).  A call's
 * layout changes it as follows:
 *   - Rows off the 128-byte grid (any tensor's rows, or the weight) run the
 *     bandwidth table's shape for their hidden: never 256 lanes x 2 (mode 0,
 *     384 < hidden / 8 <= 512: 128 x 4, flags 131 instead), the one-wave rows
 *     (modes 0, 1, 3; 384 < hidden / 8 <= 640; 768 < rows <= 2048) or the
 *     two-wave rows (modes 0, 3; 640 < hidden / 8 <= 1024; 512 < rows <=
 *     1280).  Its flags gain bit 5 (the unaligned variant; in modes 0, 1, 3
 *     and 4 it rotates each row's lane mapping onto 512-byte boundaries of
 *     the first written tensor, which changes the order in which a row's
 *     squares are summed, within the same 1-ulp bar), or bits 5 and 6 (the
 *     tail variant) for hidden % 8 != 0 and for shifted rows: modes 0-4 from
 *     hidden 4104 up when no tensor but the weight has its rows on 16-byte
 *     boundaries (plain RMSNorm with input and output at different 16-byte
 *     phases only from hidden 16384; the FP8 output only for odd hidden with
 *     every tensor at one phase).  The sc1 bits (8, 16) are dropped, except
 *     in modes 0, 1, 3 and 4 for calls of more than 2^24 elements (tail
 *     variants only past 2048 whole vectors).  The tail variant adds bit 2 to
 *     1024 x 2 and 1024 x 3, runs 1024 x 2 (flags 31, adjusted as above) in
 *     place of the LDS tier's 256 x 8, and adds bit 14 to 512 x 2-3 and
 *     1024 x 2 (modes 0, 3; from 1024 rows), 512 x 3 (mode 4; from 1024 rows)
 *     and 512 x 2-4 and 1024 x 3 (mode 1; from 384 rows).
 *   - Calls of modes 0, 2, 4, 5, 6 and 7 on the grid with rows * hidden <= 2^24
 *     whose configuration carries the sc1 bits run the same shape with flags
 *     (flags & ~24) | 32: the unaligned variant without sc1 (rows off a
 *     512-byte boundary are then rotated, as above).
 *   - Mode 0 reports bits 16-18 (row groups in runs per XCD) for hidden 4096
 *     from 4096 rows and hidden 8192 from 2048 rows, and modes 2, 5, 6 and 7
 *     for hidden 8192 from 4096 rows; calls take them when their input and
 *     residual rows are on the grid with that pitch (8 KiB, 16 KiB) and the
 *     table's shape.  Mode 7 with column-major scales (row stride 1) also
 *     takes them for hidden 4096 from 4096 rows.  Every variant above takes
 *     its row groups in the default order.
 * Pure function of its arguments; touches no device. */
int hprms_select_config(int64_t rows, int64_t hidden, int dtype, int mode, hprms_config* config);

/* hprms_select_config() for a device of `cu_count` compute units (1 ...
 * 65536).  The row-count rules above were measured on 256 CUs and depend on
 * rows per CU: on `cu_count` CUs each sees rows * 256 / cu_count rounded up,
 * and workgroup rounds are counted on `cu_count` CUs.  The entry points apply
 * it with the current device's count (hprms_device_cu_count).  With
 * cu_count = 256 it equals hprms_select_config().  No counterpart in the
 * reference, which sizes its persistent grid from the device's
 * multiProcessorCount (hp_rms_norm/csrc/cuda/hp_rms_norm.cuh:550).  Touches
 * no device. */
int hprms_select_config_cu(int64_t rows, int64_t hidden, int dtype, int mode, int cu_count,
                           hprms_config* config);

/* Compute units of HIP device `device` (< 0: the current device) as the
 * entry points use them: hipDeviceAttributeMultiprocessorCount, queried once
 * per device ordinal and cached (safe to call from any thread).  Returns the
 * count, or a negative status when the runtime cannot report it.  Replaces
 * the reference's per-call device-property query
 * (hp_rms_norm/csrc/cuda/hp_rms_norm.cuh:550,571). */
int hprms_device_cu_count(int device);

/* Batch-invariant mode, process-wide.  By default the row count selects the
 * shape (latency rows for few rows, wide, one- and two-wave rows for
 * mid-size batches: up to 29% faster there), and shapes of one width sum a
 * row's squares in different orders, so the same row can come out one ulp
 * apart in calls of different row counts (in about 1e-5 of elements; both
 * within the bar).  With the mode on, the shape follows from hidden, dtype,
 * mode and layout alone -- the bandwidth table's choice for a large batch --
 * as the reference's launcher chooses by hidden alone
 * (hp_rms_norm/csrc/cuda/hp_rms_norm.cuh:562-618), so a row's bits do not
 * depend on the call's row count; calls with few rows run slower.  Rows are
 * compared at the same addresses modulo 512 bytes (torch's allocator aligns
 * to 512): rows off the 128-byte grid take lane mappings that follow their
 * addresses.  hprms_set_batch_invariant(0 or 1) returns the previous setting
 * (or HPRMS_E_INVALID); hprms_batch_invariant() returns the current one.
 * Until set, the environment variable HPRMS_BATCH_INVARIANT=1 turns it on.
 * The setting is read once per call; hprms_select_config reports the
 * configuration under it.  No counterpart in the reference. */
int hprms_set_batch_invariant(int enable);
int hprms_batch_invariant(void);

/* Lists the vector-tier configurations built into the library for (dtype,
 * mode, numbered as for hprms_select_config).  Writes up to `capacity`
 * entries to `out` (may be NULL when capacity is 0) and returns how many
 * exist, or a negative status.  Touches no device. */
int hprms_kernel_configs(int dtype, int mode, hprms_config* out, int capacity);

/* Message of the calling thread's most recent failure ("" if none). */
const char* hprms_last_error(void);

/* HPRMS_ABI_VERSION of the built library. */
int hprms_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* HP_RMS_NORM_AMD_H_ */
