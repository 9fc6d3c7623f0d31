"""Python surface of the ops; the first two are drop-ins for the reference's
``hp_rms_norm.ops`` (hp_rms_norm/ops.py:4-24): same names, positional
argument order, in-place semantics and ``None`` return."""
import torch

__all__ = ["hp_rms_norm", "relu", "relu_max0", "rms_norm", "fused_add_rms_norm", "fused_add_rms_norm_out",
           "hp_rms_norm_fp8", "fused_add_rms_norm_fp8", "hp_rms_norm_fp8_ub", "hp_rms_norm_fp8_static",
           "fused_add_rms_norm_fp8_static",
           "hp_rms_norm_fp8_group", "fused_add_rms_norm_fp8_group",
           "reduce_add_rms_norm", "hp_rms_norm_mx",
           "fused_add_rms_norm_mxfp8", "fused_add_rms_norm_mxfp4", "MXFP8", "MXFP4",
           "set_batch_invariant", "batch_invariant"]

MXFP8, MXFP4 = 0, 1  # element formats of the OCP MX output


def hp_rms_norm(input, weight, residual, eps):
    """Fused residual-add + RMSNorm, in place (reference: hp_rms_norm/ops.py:4-15).

    ``residual <- input + residual`` (rounded to the tensor dtype) and
    ``input <- rms_norm(input + residual) * weight`` with fp32 accumulation.
    Tensors: ``input``/``residual`` [..., H] bf16 or fp16 on a HIP device,
    ``weight`` [H] of the same dtype.  Returns None.
    """
    torch.ops.hp_rms_norm.rms_norm.default(input, weight, residual, eps)


def relu(output, input):
    """The reference's "relu" (hp_rms_norm/ops.py:17-24): its kernel is an
    identity copy (activation_kernels.cuh:99-119), so ``output <- input``."""
    torch.ops.hp_rms_norm.relu.default(output, input)


def relu_max0(output, input):
    """A true ReLU on the same streamer: ``output <- max(input, 0)``,
    matching ``torch.relu`` (-0 and NaN pass through).  No reference counterpart."""
    torch.ops.hp_rms_norm.relu_max0.default(output, input)


def rms_norm(output, input, weight, eps):
    """Plain RMSNorm without a residual stream: ``output <- rms_norm(input) *
    weight``; ``output`` may be ``input``.  No reference counterpart."""
    torch.ops.hp_rms_norm.rms_norm_plain.default(output, input, weight, eps)


def fused_add_rms_norm_out(out, residual_out, input, weight, residual, eps):
    """Out-of-place ``hp_rms_norm``: ``residual_out <- input + residual`` and
    ``out <- rms_norm(residual_out) * weight``; ``input`` and ``residual`` are
    only read.  ``out`` may be ``input`` and ``residual_out`` may be
    ``residual``.  The same kernel as the in-place op (2 reads and 2 writes
    per element).  No reference counterpart."""
    torch.ops.hp_rms_norm.rms_norm_out.default(out, residual_out, input, weight, residual, eps)


def fused_add_rms_norm(input, residual, weight, eps):
    """Allocating out-of-place form of ``hp_rms_norm``: returns ``(normed,
    input + residual)`` as new tensors and leaves the arguments untouched."""
    out = torch.empty_like(input)
    res = torch.empty_like(residual)
    torch.ops.hp_rms_norm.rms_norm_out.default(out, res, input, weight, residual, eps)
    return out, res


def hp_rms_norm_fp8(output, scale, input, weight, residual, eps):
    """Fused residual-add + RMSNorm with an FP8 output, dynamic per row:
    ``residual <- input + residual`` in place; with ``y`` the op's 16-bit
    output, ``scale[r] = max(amax|y[r]| / 448, FLT_MIN)`` and ``output[r] =
    float8_e4m3fn(clamp(y[r] * (1 / scale[r]), -448, 448))``.  ``input`` is
    only read.  ``output``: float8_e4m3fn, same shape as ``input``; ``scale``:
    float32 with one element per row.  No reference counterpart."""
    torch.ops.hp_rms_norm.rms_norm_fp8_quant.default(output, scale, input, weight, residual, eps)


def fused_add_rms_norm_fp8(input, residual, weight, eps, scale_ub=None):
    """Allocating form of ``hp_rms_norm_fp8``: returns ``(q, scale)`` with
    ``q`` float8_e4m3fn shaped like ``input`` and ``scale`` float32 of shape
    ``input.shape[:-1] + (1,)``; ``residual`` is updated in place.
    ``scale_ub``: an optional one-element float32 device tensor bounding each
    row's maximum (``hp_rms_norm_fp8_ub``)."""
    q = torch.empty(input.shape, dtype=torch.float8_e4m3fn, device=input.device)
    scale = torch.empty(input.shape[:-1] + (1,), dtype=torch.float32, device=input.device)
    if scale_ub is None:
        torch.ops.hp_rms_norm.rms_norm_fp8_quant.default(q, scale, input, weight, residual, eps)
    else:
        torch.ops.hp_rms_norm.rms_norm_fp8_quant_ub.default(q, scale, input, weight, residual, scale_ub, eps)
    return q, scale


def hp_rms_norm_fp8_ub(output, scale, input, weight, residual, scale_ub, eps):
    """``hp_rms_norm_fp8`` with an upper bound on each row's maximum (the
    activation scale bound of FP8 row-wise checkpoints): ``scale = max(min(
    amax|y|, scale_ub) / 448, FLT_MIN)``, ``output`` as before with that
    scale.  ``scale_ub``: one float32 on the device, read by the kernel; a
    row holding NaN keeps a NaN scale.  No reference counterpart."""
    torch.ops.hp_rms_norm.rms_norm_fp8_quant_ub.default(output, scale, input, weight, residual, scale_ub, eps)


def hp_rms_norm_fp8_static(output, scale, input, weight, residual, eps):
    """Fused residual-add + RMSNorm with an FP8 output and one given scale for
    every row (static per-tensor quantisation): ``residual <- input +
    residual`` in place; with ``y`` the op's 16-bit output, ``output =
    float8_e4m3fn(clamp(y * (1 / scale), -448, 448))``.  ``scale``: a float32
    tensor of one element on the device, only read; ``input`` is only read.
    No reference counterpart."""
    torch.ops.hp_rms_norm.rms_norm_fp8_static_quant.default(output, scale, input, weight, residual, eps)


def fused_add_rms_norm_fp8_static(input, residual, weight, scale, eps):
    """Allocating form of ``hp_rms_norm_fp8_static``: returns ``q``
    (float8_e4m3fn shaped like ``input``); ``residual`` is updated in place."""
    q = torch.empty(input.shape, dtype=torch.float8_e4m3fn, device=input.device)
    torch.ops.hp_rms_norm.rms_norm_fp8_static_quant.default(q, scale, input, weight, residual, eps)
    return q


def hp_rms_norm_fp8_group(output, scales, input, weight, residual, eps):
    """Fused residual-add + RMSNorm with an FP8 output and one float32 scale
    per 128 consecutive elements of a row (per-token-group quantisation, 1 x
    128 groups): ``residual <- input + residual`` in place; with ``y`` the op's
    16-bit output, per group ``scales = max(amax|y| / 448, FLT_MIN)`` and
    ``output = float8_e4m3fn(clamp(y * (1 / scales), -448, 448))``.
    ``output``: float8_e4m3fn shaped like ``input``; ``scales``: float32
    ``[..., H // 128]`` with any strides under which its leading dimensions
    flatten to one row stride and no two elements share memory: rows of
    scales, or the column-major (token-minor) layout that some block-scaled
    GEMMs read, e.g. ``torch.empty(H // 128, T).t()``.  ``input`` is only
    read.  Needs ``H % 128 == 0``.  No reference counterpart."""
    torch.ops.hp_rms_norm.rms_norm_fp8_group_quant.default(output, scales, input, weight, residual, eps)


def fused_add_rms_norm_fp8_group(input, residual, weight, eps, column_major_scales=False, scale_row_align=1):
    """Allocating form of ``hp_rms_norm_fp8_group``: returns ``(q, scales)``;
    ``residual`` is updated in place.  ``column_major_scales``: the scales are
    laid out token-minor (element ``(t, g)`` at ``g * T' + t``, where ``T'``
    is the token count rounded up to a multiple of ``scale_row_align``, e.g.
    4 for 16-byte aligned columns); the returned tensor is the ``[..., H //
    128]`` view of that storage."""
    q = torch.empty(input.shape, dtype=torch.float8_e4m3fn, device=input.device)
    groups = input.shape[-1] // 128
    if column_major_scales:
        tokens = input.numel() // input.shape[-1] if input.shape[-1] else 0
        padded = -(-tokens // scale_row_align) * scale_row_align
        store = torch.empty(groups, padded, dtype=torch.float32, device=input.device)
        scales = store[:, :tokens].t().view(input.shape[:-1] + (groups,))
    else:
        scales = torch.empty(input.shape[:-1] + (groups,), dtype=torch.float32, device=input.device)
    torch.ops.hp_rms_norm.rms_norm_fp8_group_quant.default(q, scales, input, weight, residual, eps)
    return q, scales


def reduce_add_rms_norm(out, parts, weight, residual, eps):
    """Partial sums fused with ``hp_rms_norm``: with ``a = sum(parts)`` added
    in fp32 in list order and rounded once to the tensor dtype,
    ``residual <- a + residual`` in place and ``out <- rms_norm(residual) *
    weight``.  ``parts``: 1 to 8 tensors shaped like ``residual`` that share one
    row stride (the buffers of a tensor-parallel all-reduce); they are only
    read, and ``out`` may be one of them.  With one part this is
    ``hp_rms_norm`` writing its output to ``out``.  No reference counterpart."""
    torch.ops.hp_rms_norm.reduce_add_rms_norm.default(out, list(parts), weight, residual, eps)


def hp_rms_norm_mx(output, scales, input, weight, residual, eps, format):
    """Fused residual-add + RMSNorm with an OCP MX block-scaled output
    (``format`` MXFP8: E4M3 elements, MXFP4: E2M1 elements two per byte, even
    element in the low nibble).  ``residual <- input + residual`` in place;
    with ``y`` the op's 16-bit output, each block of 32 consecutive elements
    of a row gets ``scales = floor(log2(max|y|)) - emax`` as an E8M0 byte
    (emax 8 / 2; 0xFF for a block holding NaN or inf) and ``output = y / 2^s``
    rounded to nearest even, saturated.  ``output``: ``[..., H]``
    float8_e4m3fn (MXFP8) or ``[..., H // 2]`` float4_e2m1fn_x2 (MXFP4), or
    uint8; ``scales``: ``[..., H // 32]`` float8_e8m0fnu or uint8.  ``input``
    is only read.  Needs ``H % 32 == 0``.  No reference counterpart."""
    torch.ops.hp_rms_norm.rms_norm_mx_quant.default(output, scales, input, weight, residual, format, eps)


def _mx_alloc(input, format):
    h = input.shape[-1]
    if format == MXFP8:
        q = torch.empty(input.shape, dtype=torch.float8_e4m3fn, device=input.device)
    else:
        q = torch.empty(input.shape[:-1] + (h // 2,), dtype=torch.float4_e2m1fn_x2, device=input.device)
    scales = torch.empty(input.shape[:-1] + (h // 32,), dtype=torch.float8_e8m0fnu, device=input.device)
    return q, scales


def fused_add_rms_norm_mxfp8(input, residual, weight, eps):
    """Allocating MXFP8 form of ``hp_rms_norm_mx``: returns ``(q, scales)``;
    ``residual`` is updated in place."""
    q, scales = _mx_alloc(input, MXFP8)
    hp_rms_norm_mx(q, scales, input, weight, residual, eps, MXFP8)
    return q, scales


def fused_add_rms_norm_mxfp4(input, residual, weight, eps):
    """Allocating MXFP4 form of ``hp_rms_norm_mx``: returns ``(q, scales)``
    with ``q`` packed two E2M1 codes per byte; ``residual`` is updated in place."""
    q, scales = _mx_alloc(input, MXFP4)
    hp_rms_norm_mx(q, scales, input, weight, residual, eps, MXFP4)
    return q, scales


def set_batch_invariant(enable):
    """Process-wide: with ``enable`` true every call chooses its kernel shape by
    the width (and dtype, form and layout) alone, as the reference's launcher
    does (hp_rms_norm/csrc/cuda/hp_rms_norm.cuh:562-618), so a row's output
    bits do not depend on how many rows the call holds; calls with few rows
    run slower.  By default the row count also picks the shape, and the same
    row can come out one ulp apart between calls of different row counts.
    Returns the previous setting.  ``HPRMS_BATCH_INVARIANT=1`` in the
    environment turns it on until set.  No reference counterpart."""
    from . import _C
    return _C.set_batch_invariant(bool(enable))


def batch_invariant():
    """The current batch-invariant setting (see ``set_batch_invariant``)."""
    from . import _C
    return _C.batch_invariant()

