// torch_binding.cpp - registers torch.ops.hp_rms_norm.* on top of the C ABI of
// libhprms.so.  This is the only host layer between PyTorch and the kernels:
// it checks tensors, flattens them to [rows, hidden] with a row stride, picks
// the current HIP stream of the tensor's device and calls the C ABI.
//
// Schemas follow the reference's registration
// (hp_rms_norm/csrc/hp_rms_norm.cpp:35-38) with the same names and argument
// order, plus alias annotations that declare the in-place writes, so that
// functionalisation and torch.compile see them.  Messages of the shape checks
// are the reference's (hp_rms_norm/csrc/cuda/hp_rms_norm.cu:12-24,48 and
// activation_kernels.cu:11-15,38).
//
// The library is the package's importable extension module `_C`, as the
// reference's is (hp_rms_norm/__init__.py:2): importing it loads the library,
// whose static initialisers at the end of this file register the operators.
#include <Python.h>

#include <ATen/MemoryOverlap.h>
#include <ATen/core/Tensor.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include "hp_rms_norm_amd.h"

namespace {

int dtype_code(const at::Tensor& t) {
  if (t.scalar_type() == at::kBFloat16) return HPRMS_DTYPE_BF16;
  if (t.scalar_type() == at::kHalf) return HPRMS_DTYPE_FP16;
  TORCH_CHECK(false, "dtype must be kFloat16 or kBFloat16");
  return -1;
}

// Rows and row stride of a [..., hidden] tensor whose leading dims collapse
// into one (the reference flattens with view({-1, hidden}),
// hp_rms_norm/csrc/cuda/hp_rms_norm.cu:26).  Rows of width 0 hold no
// element (the ops return at once); view cannot infer their count.
void rows_of(const at::Tensor& t, int64_t hidden, int64_t* rows, int64_t* stride) {
  if (hidden == 0) {
    *rows = 1;
    for (int64_t i = 0; i + 1 < t.dim(); ++i) *rows *= t.size(i);
    *stride = 0;
    return;
  }
  at::Tensor flat = t.view({-1, hidden});
  *rows = flat.size(0);
  *stride = *rows <= 1 ? hidden : flat.stride(0);
  TORCH_CHECK(*stride >= hidden, "rows of the tensor overlap (row stride ", *stride, " < hidden ", hidden, ")");
}

void check_status(int rc) {
  TORCH_CHECK(rc == HPRMS_OK, "hp_rms_norm: ", hprms_last_error(), " (status ", rc, ")");
}

struct FusedShape {
  int64_t rows, hidden, in_stride, res_stride;
  int dtype;
};

FusedShape check_fused(const at::Tensor& input, const at::Tensor& weight, const at::Tensor& residual) {
  TORCH_CHECK(input.dim() >= 2, "input.dim() >= 2");
  TORCH_CHECK(input.dim() == residual.dim(), "input.dim() == residual.dim()");
  for (int64_t i = 0; i < input.dim(); ++i)
    TORCH_CHECK(input.size(i) == residual.size(i), "input.size(i) == residual.size(i)");
  TORCH_CHECK(weight.dim() == 1, "weight.dim() == 1");
  const int64_t hidden = weight.size(0);
  TORCH_CHECK(input.size(-1) == hidden, "input.size(-1) == hidden_dim");
  TORCH_CHECK(input.stride(-1) == 1, "input.stride(-1) == 1");
  TORCH_CHECK(residual.stride(-1) == 1, "residual.stride(-1) == 1");
  TORCH_CHECK(weight.stride(0) == 1 || hidden == 1, "weight.stride(0) == 1");
  FusedShape s;
  s.dtype = dtype_code(input);
  TORCH_CHECK(residual.scalar_type() == input.scalar_type(), "residual.dtype() == input.dtype()");
  TORCH_CHECK(weight.scalar_type() == input.scalar_type(), "weight.dtype() == input.dtype()");
  TORCH_CHECK(residual.device() == input.device() && weight.device() == input.device(),
              "input, weight and residual must be on the same device");
  s.hidden = hidden;
  rows_of(input, hidden, &s.rows, &s.in_stride);
  int64_t rrows = 0;
  rows_of(residual, hidden, &rrows, &s.res_stride);
  if (s.rows > 0) at::assert_no_overlap(input, residual);
  return s;
}

void rms_norm_hip(at::Tensor& input, const at::Tensor& weight, at::Tensor& residual, double eps) {
  const FusedShape s = check_fused(input, weight, residual);
  if (s.rows == 0 || s.hidden == 0) return;
  c10::DeviceGuard guard(input.device());
  hipStream_t stream = c10::hip::getCurrentHIPStream(input.device().index()).stream();
  check_status(hprms_fused_add_rmsnorm(input.data_ptr(), weight.data_ptr(), residual.data_ptr(), s.rows,
                                       s.hidden, s.in_stride, s.res_stride, s.dtype, eps, stream));
}

void rms_norm_meta(at::Tensor& input, const at::Tensor& weight, at::Tensor& residual, double eps) {
  (void)check_fused(input, weight, residual);
  (void)eps;
}

struct StreamShape {
  int64_t rows, hidden, out_stride, in_stride;
  int dtype;
};

StreamShape check_stream(const at::Tensor& out, const at::Tensor& input) {
  TORCH_CHECK(input.dim() >= 2, "input.dim() >= 2");
  TORCH_CHECK(input.dim() == out.dim(), "input.dim() == out.dim()");
  for (int64_t i = 0; i < input.dim(); ++i)
    TORCH_CHECK(input.size(i) == out.size(i), "input.size(i) == out.size(i)");
  TORCH_CHECK(input.stride(-1) == 1, "input.stride(-1) == 1");
  TORCH_CHECK(out.stride(-1) == 1, "out.stride(-1) == 1");
  StreamShape s;
  s.dtype = dtype_code(input);
  TORCH_CHECK(out.scalar_type() == input.scalar_type(), "out.dtype() == input.dtype()");
  TORCH_CHECK(out.device() == input.device(), "out and input must be on the same device");
  s.hidden = input.size(-1);
  int64_t orows = 0;
  rows_of(input, s.hidden, &s.rows, &s.in_stride);
  rows_of(out, s.hidden, &orows, &s.out_stride);
  if (s.rows > 0 && s.hidden > 0) at::assert_no_partial_overlap(out, input);
  return s;
}

void stream_hip(at::Tensor& out, const at::Tensor& input, int op) {
  const StreamShape s = check_stream(out, input);
  if (s.rows == 0 || s.hidden == 0) return;
  c10::DeviceGuard guard(input.device());
  hipStream_t stream = c10::hip::getCurrentHIPStream(input.device().index()).stream();
  check_status(hprms_streamer(out.data_ptr(), input.data_ptr(), s.rows, s.hidden, s.out_stride, s.in_stride,
                              s.dtype, op, stream));
}

void relu_hip(at::Tensor& out, const at::Tensor& input) { stream_hip(out, input, HPRMS_STREAM_COPY); }
void relu_max0_hip(at::Tensor& out, const at::Tensor& input) { stream_hip(out, input, HPRMS_STREAM_RELU); }
void stream_meta(at::Tensor& out, const at::Tensor& input) { (void)check_stream(out, input); }

struct PlainShape {
  int64_t rows, hidden, out_stride, in_stride;
  int dtype;
};

PlainShape check_plain(const at::Tensor& out, const at::Tensor& input, const at::Tensor& weight) {
  TORCH_CHECK(input.dim() >= 2, "input.dim() >= 2");
  TORCH_CHECK(input.dim() == out.dim(), "input.dim() == out.dim()");
  for (int64_t i = 0; i < input.dim(); ++i)
    TORCH_CHECK(input.size(i) == out.size(i), "input.size(i) == out.size(i)");
  TORCH_CHECK(weight.dim() == 1, "weight.dim() == 1");
  const int64_t hidden = weight.size(0);
  TORCH_CHECK(input.size(-1) == hidden, "input.size(-1) == hidden_dim");
  TORCH_CHECK(input.stride(-1) == 1, "input.stride(-1) == 1");
  TORCH_CHECK(out.stride(-1) == 1, "out.stride(-1) == 1");
  TORCH_CHECK(weight.stride(0) == 1 || hidden == 1, "weight.stride(0) == 1");
  PlainShape s;
  s.dtype = dtype_code(input);
  TORCH_CHECK(out.scalar_type() == input.scalar_type(), "out.dtype() == input.dtype()");
  TORCH_CHECK(weight.scalar_type() == input.scalar_type(), "weight.dtype() == input.dtype()");
  TORCH_CHECK(out.device() == input.device() && weight.device() == input.device(),
              "out, input and weight must be on the same device");
  s.hidden = hidden;
  int64_t orows = 0;
  rows_of(input, hidden, &s.rows, &s.in_stride);
  rows_of(out, hidden, &orows, &s.out_stride);
  if (s.rows > 0) at::assert_no_partial_overlap(out, input);
  return s;
}

void rms_norm_plain_hip(at::Tensor& out, const at::Tensor& input, const at::Tensor& weight, double eps) {
  const PlainShape s = check_plain(out, input, weight);
  if (s.rows == 0 || s.hidden == 0) return;
  c10::DeviceGuard guard(input.device());
  hipStream_t stream = c10::hip::getCurrentHIPStream(input.device().index()).stream();
  check_status(hprms_rmsnorm(out.data_ptr(), input.data_ptr(), weight.data_ptr(), s.rows, s.hidden,
                             s.out_stride, s.in_stride, s.dtype, eps, stream));
}

void rms_norm_plain_meta(at::Tensor& out, const at::Tensor& input, const at::Tensor& weight, double eps) {
  (void)check_plain(out, input, weight);
  (void)eps;
}

struct Fp8Shape {
  FusedShape f;
  int64_t out_stride;
};

Fp8Shape check_fp8(const at::Tensor& out, const at::Tensor& scale, const at::Tensor& input,
                   const at::Tensor& weight, const at::Tensor& residual) {
  Fp8Shape s;
  s.f = check_fused(input, weight, residual);
  TORCH_CHECK(out.scalar_type() == at::kFloat8_e4m3fn, "out.dtype() == float8_e4m3fn");
  TORCH_CHECK(scale.scalar_type() == at::kFloat, "scale.dtype() == float32");
  TORCH_CHECK(out.dim() == input.dim(), "out.dim() == input.dim()");
  for (int64_t i = 0; i < input.dim(); ++i) TORCH_CHECK(out.size(i) == input.size(i), "out.size(i) == input.size(i)");
  TORCH_CHECK(out.stride(-1) == 1, "out.stride(-1) == 1");
  TORCH_CHECK(scale.numel() == s.f.rows, "scale.numel() == number of rows");
  TORCH_CHECK(scale.is_contiguous(), "scale must be contiguous");
  TORCH_CHECK(out.device() == input.device() && scale.device() == input.device(),
              "out, scale and input must be on the same device");
  int64_t orows = 0;
  rows_of(out, s.f.hidden, &orows, &s.out_stride);
  if (s.f.rows > 0) {
    // the FP8 rows and the scales are written while input and residual are
    // read: no sharing between any two of them
    at::assert_no_overlap(out, residual);
    at::assert_no_overlap(out, input);
    at::assert_no_overlap(scale, residual);
    at::assert_no_overlap(scale, input);
    at::assert_no_overlap(scale, out);
  }
  return s;
}

void rms_norm_fp8_hip(at::Tensor& out, at::Tensor& scale, const at::Tensor& input, const at::Tensor& weight,
                      at::Tensor& residual, double eps) {
  const Fp8Shape s = check_fp8(out, scale, input, weight, residual);
  if (s.f.rows == 0 || s.f.hidden == 0) return;
  c10::DeviceGuard guard(input.device());
  hipStream_t stream = c10::hip::getCurrentHIPStream(input.device().index()).stream();
  check_status(hprms_fused_add_rmsnorm_fp8(out.data_ptr(), scale.data_ptr<float>(), input.data_ptr(),
                                           weight.data_ptr(), residual.data_ptr(), s.f.rows, s.f.hidden,
                                           s.out_stride, s.f.in_stride, s.f.res_stride, s.f.dtype, eps, stream));
}

void rms_norm_fp8_meta(at::Tensor& out, at::Tensor& scale, const at::Tensor& input, const at::Tensor& weight,
                       at::Tensor& residual, double eps) {
  (void)check_fp8(out, scale, input, weight, residual);
  (void)eps;
}

// ---- FP8 output with per-row scales bounded above ------------------------------------
Fp8Shape check_fp8_ub(const at::Tensor& out, const at::Tensor& scale, const at::Tensor& input,
                      const at::Tensor& weight, const at::Tensor& residual, const at::Tensor& scale_ub) {
  const Fp8Shape s = check_fp8(out, scale, input, weight, residual);
  TORCH_CHECK(scale_ub.scalar_type() == at::kFloat, "scale_ub.dtype() == float32");
  TORCH_CHECK(scale_ub.numel() == 1, "scale_ub must hold one element");
  TORCH_CHECK(scale_ub.device() == input.device(), "scale_ub and input must be on the same device");
  if (s.f.rows > 0) at::assert_no_overlap(scale, scale_ub);
  return s;
}

void rms_norm_fp8_ub_hip(at::Tensor& out, at::Tensor& scale, const at::Tensor& input, const at::Tensor& weight,
                         at::Tensor& residual, const at::Tensor& scale_ub, double eps) {
  const Fp8Shape s = check_fp8_ub(out, scale, input, weight, residual, scale_ub);
  if (s.f.rows == 0 || s.f.hidden == 0) return;
  c10::DeviceGuard guard(input.device());
  hipStream_t stream = c10::hip::getCurrentHIPStream(input.device().index()).stream();
  check_status(hprms_fused_add_rmsnorm_fp8_ub(out.data_ptr(), scale.data_ptr<float>(), scale_ub.data_ptr<float>(),
                                              input.data_ptr(), weight.data_ptr(), residual.data_ptr(), s.f.rows,
                                              s.f.hidden, s.out_stride, s.f.in_stride, s.f.res_stride, s.f.dtype,
                                              eps, stream));
}

void rms_norm_fp8_ub_meta(at::Tensor& out, at::Tensor& scale, const at::Tensor& input, const at::Tensor& weight,
                          at::Tensor& residual, const at::Tensor& scale_ub, double eps) {
  (void)check_fp8_ub(out, scale, input, weight, residual, scale_ub);
  (void)eps;
}

// ---- FP8 output with one given scale ---------------------------------------------------
Fp8Shape check_fp8_static(const at::Tensor& out, const at::Tensor& scale, const at::Tensor& input,
                          const at::Tensor& weight, const at::Tensor& residual) {
  Fp8Shape s;
  s.f = check_fused(input, weight, residual);
  TORCH_CHECK(out.scalar_type() == at::kFloat8_e4m3fn, "out.dtype() == float8_e4m3fn");
  TORCH_CHECK(scale.scalar_type() == at::kFloat, "scale.dtype() == float32");
  TORCH_CHECK(scale.numel() == 1, "scale must hold one element (one scale for every row)");
  TORCH_CHECK(out.dim() == input.dim(), "out.dim() == input.dim()");
  for (int64_t i = 0; i < input.dim(); ++i) TORCH_CHECK(out.size(i) == input.size(i), "out.size(i) == input.size(i)");
  TORCH_CHECK(out.stride(-1) == 1, "out.stride(-1) == 1");
  TORCH_CHECK(out.device() == input.device() && scale.device() == input.device(),
              "out, scale and input must be on the same device");
  int64_t orows = 0;
  rows_of(out, s.f.hidden, &orows, &s.out_stride);
  if (s.f.rows > 0) {
    // the FP8 rows are written while input, residual and the scale are read
    at::assert_no_overlap(out, residual);
    at::assert_no_overlap(out, input);
    at::assert_no_overlap(out, scale);
    at::assert_no_overlap(residual, scale);
  }
  return s;
}

void rms_norm_fp8_static_hip(at::Tensor& out, const at::Tensor& scale, const at::Tensor& input,
                             const at::Tensor& weight, at::Tensor& residual, double eps) {
  const Fp8Shape s = check_fp8_static(out, scale, input, weight, residual);
  if (s.f.rows == 0 || s.f.hidden == 0) return;
  c10::DeviceGuard guard(input.device());
  hipStream_t stream = c10::hip::getCurrentHIPStream(input.device().index()).stream();
  check_status(hprms_fused_add_rmsnorm_fp8_static(out.data_ptr(), scale.data_ptr<float>(), input.data_ptr(),
                                                  weight.data_ptr(), residual.data_ptr(), s.f.rows, s.f.hidden,
                                                  s.out_stride, s.f.in_stride, s.f.res_stride, s.f.dtype, eps,
                                                  stream));
}

void rms_norm_fp8_static_meta(at::Tensor& out, const at::Tensor& scale, const at::Tensor& input,
                              const at::Tensor& weight, at::Tensor& residual, double eps) {
  (void)check_fp8_static(out, scale, input, weight, residual);
  (void)eps;
}

// ---- FP8 output with a scale per 128 elements -------------------------------------------
struct GroupShape {
  FusedShape f;
  int64_t out_stride, scale_stride, scale_group_stride;
};

GroupShape check_fp8_group(const at::Tensor& out, const at::Tensor& scales, const at::Tensor& input,
                           const at::Tensor& weight, const at::Tensor& residual) {
  GroupShape s;
  s.f = check_fused(input, weight, residual);
  TORCH_CHECK(s.f.hidden % 128 == 0, "the FP8 output with a scale per 128 elements needs hidden_dim % 128 == 0");
  TORCH_CHECK(out.scalar_type() == at::kFloat8_e4m3fn, "out.dtype() == float8_e4m3fn");
  TORCH_CHECK(scales.scalar_type() == at::kFloat, "scales.dtype() == float32");
  for (const at::Tensor* t : {&out, &scales}) {
    TORCH_CHECK(t->dim() == input.dim(), "out and scales must have input.dim() dimensions");
    for (int64_t i = 0; i + 1 < input.dim(); ++i)
      TORCH_CHECK(t->size(i) == input.size(i), "out and scales must match input in the leading dimensions");
    TORCH_CHECK(t->device() == input.device(), "out, scales and input must be on the same device");
  }
  TORCH_CHECK(out.stride(-1) == 1, "out must be contiguous in the last dimension");
  TORCH_CHECK(out.size(-1) == s.f.hidden, "out.size(-1) == hidden_dim");
  TORCH_CHECK(scales.size(-1) == s.f.hidden / 128, "scales.size(-1) must be hidden / 128 = ", s.f.hidden / 128);
  int64_t r = 0;
  rows_of(out, s.f.hidden, &r, &s.out_stride);
  // scales: rows of scales or the column-major (token-minor) layout; the
  // leading dimensions must flatten to one row stride, and the C ABI rejects
  // strides under which two (row, group) pairs share a scale
  TORCH_CHECK(at::has_internal_overlap(scales) != at::MemOverlap::Yes, "scales must not overlap themselves");
  s.scale_stride = 0;
  s.scale_group_stride = 1;
  if (s.f.hidden > 0) {
    const at::Tensor flat = scales.view({-1, s.f.hidden / 128});
    s.scale_stride = flat.size(0) <= 1 ? s.f.hidden / 128 : flat.stride(0);
    s.scale_group_stride = flat.size(1) <= 1 ? 1 : flat.stride(1);
  }
  if (s.f.rows > 0) {
    at::assert_no_overlap(out, scales);
    at::assert_no_overlap(out, residual);
    at::assert_no_overlap(out, input);
    at::assert_no_overlap(scales, residual);
    at::assert_no_overlap(scales, input);
  }
  return s;
}

void rms_norm_fp8_group_hip(at::Tensor& out, at::Tensor& scales, const at::Tensor& input, const at::Tensor& weight,
                            at::Tensor& residual, double eps) {
  const GroupShape s = check_fp8_group(out, scales, input, weight, residual);
  if (s.f.rows == 0 || s.f.hidden == 0) return;
  c10::DeviceGuard guard(input.device());
  hipStream_t stream = c10::hip::getCurrentHIPStream(input.device().index()).stream();
  check_status(hprms_fused_add_rmsnorm_fp8_group(out.data_ptr(), scales.data_ptr<float>(), input.data_ptr(),
                                                 weight.data_ptr(), residual.data_ptr(), s.f.rows, s.f.hidden,
                                                 s.out_stride, s.scale_stride, s.scale_group_stride,
                                                 s.f.in_stride, s.f.res_stride, s.f.dtype, eps, stream));
}

void rms_norm_fp8_group_meta(at::Tensor& out, at::Tensor& scales, const at::Tensor& input, const at::Tensor& weight,
                             at::Tensor& residual, double eps) {
  (void)check_fp8_group(out, scales, input, weight, residual);
  (void)eps;
}

// ---- fused op out of place ----------------------------------------------------------
FusedShape check_fused_out(const at::Tensor& out, const at::Tensor& residual_out, const at::Tensor& input,
                           const at::Tensor& weight, const at::Tensor& residual) {
  TORCH_CHECK(input.dim() >= 2, "input.dim() >= 2");
  const int64_t hidden = weight.dim() == 1 ? weight.size(0) : -1;
  for (const at::Tensor* t : {&residual, &out, &residual_out}) {
    TORCH_CHECK(t->dim() == input.dim(), "all row tensors must have input.dim() dimensions");
    for (int64_t i = 0; i < input.dim(); ++i) TORCH_CHECK(t->size(i) == input.size(i), "input.size(i) == residual.size(i)");
    TORCH_CHECK(t->stride(-1) == 1, "rows must be contiguous (stride(-1) == 1)");
    TORCH_CHECK(t->scalar_type() == input.scalar_type(), "all tensors must have input.dtype()");
    TORCH_CHECK(t->device() == input.device(), "all tensors must be on input's device");
  }
  TORCH_CHECK(weight.dim() == 1, "weight.dim() == 1");
  TORCH_CHECK(input.size(-1) == hidden, "input.size(-1) == hidden_dim");
  TORCH_CHECK(input.stride(-1) == 1, "input.stride(-1) == 1");
  TORCH_CHECK(weight.stride(0) == 1 || hidden == 1, "weight.stride(0) == 1");
  TORCH_CHECK(weight.scalar_type() == input.scalar_type(), "weight.dtype() == input.dtype()");
  TORCH_CHECK(weight.device() == input.device(), "weight must be on input's device");
  FusedShape s;
  s.dtype = dtype_code(input);
  s.hidden = hidden;
  rows_of(input, hidden, &s.rows, &s.in_stride);
  int64_t r = 0, st = 0;
  rows_of(residual, hidden, &r, &s.res_stride);
  rows_of(out, hidden, &r, &st);
  rows_of(residual_out, hidden, &r, &st);
  if (s.rows > 0) {
    // out may be input and residual_out may be residual (in place); no other sharing
    at::assert_no_overlap(out, residual_out);
    at::assert_no_overlap(out, residual);
    at::assert_no_overlap(residual_out, input);
    at::assert_no_partial_overlap(out, input);
    at::assert_no_partial_overlap(residual_out, residual);
  }
  return s;
}

void rms_norm_out_hip(at::Tensor& out, at::Tensor& residual_out, const at::Tensor& input, const at::Tensor& weight,
                      const at::Tensor& residual, double eps) {
  const FusedShape s = check_fused_out(out, residual_out, input, weight, residual);
  if (s.rows == 0 || s.hidden == 0) return;
  int64_t r = 0, out_stride = 0, res_out_stride = 0;
  rows_of(out, s.hidden, &r, &out_stride);
  rows_of(residual_out, s.hidden, &r, &res_out_stride);
  c10::DeviceGuard guard(input.device());
  hipStream_t stream = c10::hip::getCurrentHIPStream(input.device().index()).stream();
  check_status(hprms_fused_add_rmsnorm_out(out.data_ptr(), residual_out.data_ptr(), input.data_ptr(),
                                           residual.data_ptr(), weight.data_ptr(), s.rows, s.hidden, out_stride,
                                           res_out_stride, s.in_stride, s.res_stride, s.dtype, eps, stream));
}

void rms_norm_out_meta(at::Tensor& out, at::Tensor& residual_out, const at::Tensor& input, const at::Tensor& weight,
                       const at::Tensor& residual, double eps) {
  (void)check_fused_out(out, residual_out, input, weight, residual);
  (void)eps;
}

// ---- partial-sum reduction + fused op ----------------------------------------------------
struct ReduceShape {
  int64_t rows, hidden, out_stride, part_stride, res_stride;
  int dtype;
};

ReduceShape check_reduce(const at::Tensor& out, at::TensorList parts, const at::Tensor& weight,
                         const at::Tensor& residual) {
  TORCH_CHECK(!parts.empty() && (int64_t)parts.size() <= HPRMS_MAX_PARTS, "parts must hold 1 to ",
              HPRMS_MAX_PARTS, " tensors (got ", parts.size(), ")");
  TORCH_CHECK(residual.dim() >= 2, "input.dim() >= 2");
  TORCH_CHECK(weight.dim() == 1, "weight.dim() == 1");
  const int64_t hidden = weight.size(0);
  TORCH_CHECK(residual.size(-1) == hidden, "input.size(-1) == hidden_dim");
  TORCH_CHECK(weight.stride(0) == 1 || hidden == 1, "weight.stride(0) == 1");
  ReduceShape s;
  s.dtype = dtype_code(residual);
  s.hidden = hidden;
  TORCH_CHECK(weight.scalar_type() == residual.scalar_type(), "weight.dtype() == input.dtype()");
  TORCH_CHECK(weight.device() == residual.device(), "weight must be on residual's device");
  for (const at::Tensor* t : {&out, &parts[0]}) {
    TORCH_CHECK(t->dim() == residual.dim(), "all row tensors must have residual.dim() dimensions");
    for (int64_t i = 0; i < residual.dim(); ++i)
      TORCH_CHECK(t->size(i) == residual.size(i), "input.size(i) == residual.size(i)");
  }
  for (const at::Tensor* t : {&residual, &out}) {
    TORCH_CHECK(t->stride(-1) == 1, "rows must be contiguous (stride(-1) == 1)");
    TORCH_CHECK(t->scalar_type() == residual.scalar_type(), "all tensors must have residual.dtype()");
    TORCH_CHECK(t->device() == residual.device(), "all tensors must be on residual's device");
  }
  rows_of(residual, hidden, &s.rows, &s.res_stride);
  int64_t r = 0;
  rows_of(out, hidden, &r, &s.out_stride);
  for (size_t g = 0; g < parts.size(); ++g) {
    const at::Tensor& p = parts[g];
    TORCH_CHECK(p.sizes() == parts[0].sizes(), "every part must have the shape of the residual");
    TORCH_CHECK(p.stride(-1) == 1, "rows must be contiguous (stride(-1) == 1)");
    TORCH_CHECK(p.scalar_type() == residual.scalar_type(), "all tensors must have residual.dtype()");
    TORCH_CHECK(p.device() == residual.device(), "all tensors must be on residual's device");
    int64_t st = 0;
    rows_of(p, hidden, &r, &st);
    if (g == 0) s.part_stride = st;
    TORCH_CHECK(st == s.part_stride, "all parts must share one row stride");
    if (s.rows > 0) {
      at::assert_no_overlap(p, residual);
      at::assert_no_partial_overlap(out, p);
    }
  }
  if (s.rows > 0) at::assert_no_overlap(out, residual);
  return s;
}

void reduce_rms_norm_hip(at::Tensor& out, at::TensorList parts, const at::Tensor& weight, at::Tensor& residual,
                         double eps) {
  const ReduceShape s = check_reduce(out, parts, weight, residual);
  if (s.rows == 0 || s.hidden == 0) return;
  const void* ptrs[HPRMS_MAX_PARTS];
  for (size_t g = 0; g < parts.size(); ++g) ptrs[g] = parts[g].data_ptr();
  c10::DeviceGuard guard(residual.device());
  hipStream_t stream = c10::hip::getCurrentHIPStream(residual.device().index()).stream();
  check_status(hprms_reduce_add_rmsnorm(out.data_ptr(), ptrs, (int)parts.size(), weight.data_ptr(),
                                        residual.data_ptr(), s.rows, s.hidden, s.out_stride, s.part_stride,
                                        s.res_stride, s.dtype, eps, stream));
}

void reduce_rms_norm_meta(at::Tensor& out, at::TensorList parts, const at::Tensor& weight, at::Tensor& residual,
                          double eps) {
  (void)check_reduce(out, parts, weight, residual);
  (void)eps;
}

// ---- fused op with an OCP MX output ---------------------------------------------------
struct MxShape {
  FusedShape f;
  int64_t out_stride, scale_stride;
};

MxShape check_mx(const at::Tensor& out, const at::Tensor& scales, const at::Tensor& input, const at::Tensor& weight,
                 const at::Tensor& residual, int64_t format) {
  TORCH_CHECK(format == HPRMS_MX_FP8_E4M3 || format == HPRMS_MX_FP4_E2M1,
              "format must be 0 (MXFP8, E4M3) or 1 (MXFP4, E2M1)");
  MxShape s;
  s.f = check_fused(input, weight, residual);
  TORCH_CHECK(s.f.hidden % 32 == 0, "MX output needs hidden_dim % 32 == 0");
  const bool fp8 = format == HPRMS_MX_FP8_E4M3;
  TORCH_CHECK(out.scalar_type() == at::kByte ||
                  out.scalar_type() == (fp8 ? at::kFloat8_e4m3fn : at::kFloat4_e2m1fn_x2),
              fp8 ? "out.dtype() must be float8_e4m3fn or uint8" : "out.dtype() must be float4_e2m1fn_x2 or uint8");
  TORCH_CHECK(scales.scalar_type() == at::kByte || scales.scalar_type() == at::kFloat8_e8m0fnu,
              "scales.dtype() must be float8_e8m0fnu or uint8");
  const int64_t qw = fp8 ? s.f.hidden : s.f.hidden / 2;
  for (const at::Tensor* t : {&out, &scales}) {
    TORCH_CHECK(t->dim() == input.dim(), "out and scales must have input.dim() dimensions");
    for (int64_t i = 0; i + 1 < input.dim(); ++i)
      TORCH_CHECK(t->size(i) == input.size(i), "out and scales must match input in the leading dimensions");
    TORCH_CHECK(t->stride(-1) == 1, "out and scales must be contiguous in the last dimension");
    TORCH_CHECK(t->device() == input.device(), "out, scales and input must be on the same device");
  }
  TORCH_CHECK(out.size(-1) == qw, "out.size(-1) must be ", qw, " (", fp8 ? "hidden" : "hidden / 2", ")");
  TORCH_CHECK(scales.size(-1) == s.f.hidden / 32, "scales.size(-1) must be hidden / 32 = ", s.f.hidden / 32);
  int64_t r = 0;
  rows_of(out, qw, &r, &s.out_stride);
  rows_of(scales, s.f.hidden / 32, &r, &s.scale_stride);
  if (s.f.rows > 0) {
    at::assert_no_overlap(out, scales);
    at::assert_no_overlap(out, residual);
    at::assert_no_overlap(out, input);
    at::assert_no_overlap(scales, residual);
    at::assert_no_overlap(scales, input);
  }
  return s;
}

void rms_norm_mx_hip(at::Tensor& out, at::Tensor& scales, const at::Tensor& input, const at::Tensor& weight,
                     at::Tensor& residual, int64_t format, double eps) {
  const MxShape s = check_mx(out, scales, input, weight, residual, format);
  if (s.f.rows == 0 || s.f.hidden == 0) return;
  c10::DeviceGuard guard(input.device());
  hipStream_t stream = c10::hip::getCurrentHIPStream(input.device().index()).stream();
  check_status(hprms_fused_add_rmsnorm_mx(out.data_ptr(), scales.data_ptr(), input.data_ptr(), weight.data_ptr(),
                                          residual.data_ptr(), s.f.rows, s.f.hidden, s.out_stride, s.scale_stride,
                                          s.f.in_stride, s.f.res_stride, (int)format, s.f.dtype, eps, stream));
}

void rms_norm_mx_meta(at::Tensor& out, at::Tensor& scales, const at::Tensor& input, const at::Tensor& weight,
                      at::Tensor& residual, int64_t format, double eps) {
  (void)check_mx(out, scales, input, weight, residual, format);
  (void)eps;
}

// _C.set_batch_invariant(enable) -> previous setting; _C.batch_invariant()
// -> current setting (hprms_set_batch_invariant / hprms_batch_invariant).
PyObject* py_set_batch_invariant(PyObject*, PyObject* arg) {
  const int on = PyObject_IsTrue(arg);
  if (on < 0) return nullptr;
  const int previous = hprms_set_batch_invariant(on);
  if (previous < 0) {
    PyErr_SetString(PyExc_RuntimeError, hprms_last_error());
    return nullptr;
  }
  return PyBool_FromLong(previous);
}

PyObject* py_batch_invariant(PyObject*, PyObject*) { return PyBool_FromLong(hprms_batch_invariant()); }

PyMethodDef kMethods[] = {
    {"set_batch_invariant", py_set_batch_invariant, METH_O,
     "set_batch_invariant(enable) -> bool: choose each call's kernel shape by the width alone (a row's bits "
     "then do not depend on the call's row count); returns the previous setting"},
    {"batch_invariant", py_batch_invariant, METH_NOARGS, "batch_invariant() -> bool: the current setting"},
    {nullptr, nullptr, 0, nullptr}};

}  // namespace

// Module init of `hp_rms_norm_amd._C`.  The operators live in torch's
// registry, so the module itself carries the C ABI version it was built
// against and the batch-invariant mode's setter and getter.
extern "C" PyObject* PyInit__C(void) {
  static PyModuleDef def = {PyModuleDef_HEAD_INIT, "_C",
                            "torch.ops.hp_rms_norm.* on the gfx950 kernels of libhprms.so", -1, kMethods};
  PyObject* m = PyModule_Create(&def);
  if (m && PyModule_AddIntConstant(m, "abi_version", hprms_abi_version()) != 0) {
    Py_DECREF(m);
    return nullptr;
  }
  return m;
}

TORCH_LIBRARY(hp_rms_norm, m) {
  m.def("rms_norm(Tensor(a!) input, Tensor weight, Tensor(b!) residual, float eps) -> ()");
  m.def("relu(Tensor(a!) out, Tensor input) -> ()");
  m.def("relu_max0(Tensor(a!) out, Tensor input) -> ()");
  m.def("rms_norm_plain(Tensor(a!) out, Tensor input, Tensor weight, float eps) -> ()");
  m.def("rms_norm_fp8_quant(Tensor(a!) out, Tensor(b!) scale, Tensor input, Tensor weight, Tensor(c!) residual, "
        "float eps) -> ()");
  m.def("rms_norm_fp8_quant_ub(Tensor(a!) out, Tensor(b!) scale, Tensor input, Tensor weight, Tensor(c!) residual, "
        "Tensor scale_ub, float eps) -> ()");
  m.def("rms_norm_fp8_static_quant(Tensor(a!) out, Tensor scale, Tensor input, Tensor weight, Tensor(b!) residual, "
        "float eps) -> ()");
  m.def("rms_norm_fp8_group_quant(Tensor(a!) out, Tensor(b!) scales, Tensor input, Tensor weight, "
        "Tensor(c!) residual, float eps) -> ()");
  m.def("rms_norm_out(Tensor(a!) out, Tensor(b!) residual_out, Tensor input, Tensor weight, Tensor residual, "
        "float eps) -> ()");
  m.def("reduce_add_rms_norm(Tensor(a!) out, Tensor[] parts, Tensor weight, Tensor(b!) residual, float eps) -> ()");
  m.def("rms_norm_mx_quant(Tensor(a!) out, Tensor(b!) scales, Tensor input, Tensor weight, Tensor(c!) residual, "
        "int format, float eps) -> ()");
}

// ROCm builds of PyTorch expose HIP devices under the CUDA dispatch key.
TORCH_LIBRARY_IMPL(hp_rms_norm, CUDA, m) {
  m.impl("rms_norm", &rms_norm_hip);
  m.impl("relu", &relu_hip);
  m.impl("relu_max0", &relu_max0_hip);
  m.impl("rms_norm_plain", &rms_norm_plain_hip);
  m.impl("rms_norm_fp8_quant", &rms_norm_fp8_hip);
  m.impl("rms_norm_fp8_quant_ub", &rms_norm_fp8_ub_hip);
  m.impl("rms_norm_fp8_static_quant", &rms_norm_fp8_static_hip);
  m.impl("rms_norm_fp8_group_quant", &rms_norm_fp8_group_hip);
  m.impl("rms_norm_out", &rms_norm_out_hip);
  m.impl("reduce_add_rms_norm", &reduce_rms_norm_hip);
  m.impl("rms_norm_mx_quant", &rms_norm_mx_hip);
}

// Shape checks only, for fake tensors / torch.compile tracing.  Meta tensors
// carry no data, so nothing is computed here.
TORCH_LIBRARY_IMPL(hp_rms_norm, Meta, m) {
  m.impl("rms_norm", &rms_norm_meta);
  m.impl("relu", &stream_meta);
  m.impl("relu_max0", &stream_meta);
  m.impl("rms_norm_plain", &rms_norm_plain_meta);
  m.impl("rms_norm_fp8_quant", &rms_norm_fp8_meta);
  m.impl("rms_norm_fp8_quant_ub", &rms_norm_fp8_ub_meta);
  m.impl("rms_norm_fp8_static_quant", &rms_norm_fp8_static_meta);
  m.impl("rms_norm_fp8_group_quant", &rms_norm_fp8_group_meta);
  m.impl("rms_norm_out", &rms_norm_out_meta);
  m.impl("reduce_add_rms_norm", &reduce_rms_norm_meta);
  m.impl("rms_norm_mx_quant", &rms_norm_mx_meta);
}
