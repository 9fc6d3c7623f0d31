"""The torch binding, on the CPU: schemas, the drop-in Python surface, the
reference's shape checks and messages (hp_rms_norm/csrc/cuda/hp_rms_norm.cu:12-24,48,
activation_kernels.cu:11-15) exercised through the Meta kernels, and no CPU
fallback (CPU tensors are refused by the dispatcher)."""
import inspect
import os

import pytest
import torch

import hp_rms_norm_amd
from hp_rms_norm_amd import ops

M = "meta"


def t(*shape, dtype=torch.bfloat16):
    return torch.empty(*shape, dtype=dtype, device=M)


def test_schemas_keep_reference_names_and_order_with_alias_annotations():
    s = str(torch.ops.hp_rms_norm.rms_norm.default._schema)
    assert s == "hp_rms_norm::rms_norm(Tensor(a!) input, Tensor weight, Tensor(b!) residual, float eps) -> ()"
    s = str(torch.ops.hp_rms_norm.relu.default._schema)
    assert s == "hp_rms_norm::relu(Tensor(a!) out, Tensor input) -> ()"


def test_python_surface_matches_reference_ops():
    # hp_rms_norm/ops.py:4-24
    assert list(inspect.signature(ops.hp_rms_norm).parameters) == ["input", "weight", "residual", "eps"]
    assert list(inspect.signature(ops.relu).parameters) == ["output", "input"]
    import hp_rms_norm  # the import-compatible alias package
    assert hp_rms_norm.hp_rms_norm is ops.hp_rms_norm and hp_rms_norm.relu is ops.relu
    assert hp_rms_norm.ops.hp_rms_norm is ops.hp_rms_norm


def test_reference_import_paths():
    """Every import form of the reference package works on the alias
    (hp_rms_norm/__init__.py:1-3, hp_rms_norm/ops.py:1-24): the ``ops``
    submodule and ``_C``, the extension module whose import registers the ops."""
    import importlib
    import types

    import hp_rms_norm
    import hp_rms_norm.ops
    from hp_rms_norm import _C
    from hp_rms_norm.ops import hp_rms_norm as f, relu
    c2 = importlib.import_module("hp_rms_norm._C")
    assert f is ops.hp_rms_norm and relu is ops.relu
    assert hp_rms_norm.ops.hp_rms_norm is ops.hp_rms_norm and hp_rms_norm.ops.relu is ops.relu
    assert isinstance(_C, types.ModuleType) and c2 is _C and _C is hp_rms_norm_amd._C
    assert os.path.samefile(_C.__file__, hp_rms_norm_amd.TORCH_LIB)
    from hp_rms_norm_amd import abi
    assert _C.abi_version == abi.lib().hprms_abi_version()


def test_meta_accepts_valid_shapes():
    assert ops.hp_rms_norm(t(4, 4096), t(4096), t(4, 4096), 1e-6) is None
    assert ops.hp_rms_norm(t(2, 3, 128), t(128), t(2, 3, 128), 1e-6) is None
    assert ops.relu(t(4, 256), t(4, 256)) is None
    assert ops.relu_max0(t(4, 256, dtype=torch.float16), t(4, 256, dtype=torch.float16)) is None
    assert ops.rms_norm(t(4, 256), t(4, 256), t(256), 1e-6) is None


@pytest.mark.parametrize("args,msg", [
    ((t(4096), t(4096), t(4096)), r"input.dim\(\) >= 2"),
    ((t(4, 4096), t(4096), t(1, 4, 4096)), r"input.dim\(\) == residual.dim\(\)"),
    ((t(4, 4096), t(4096), t(5, 4096)), r"input.size\(i\) == residual.size\(i\)"),
    ((t(4, 4096), t(1, 4096), t(4, 4096)), r"weight.dim\(\) == 1"),
    ((t(4, 4096), t(2048), t(4, 4096)), r"input.size\(-1\) == hidden_dim"),
    ((t(4096, 4).t(), t(4096), t(4, 4096)), r"input.stride\(-1\) == 1"),
    ((t(4, 4096), t(4096), t(4096, 4).t()), r"residual.stride\(-1\) == 1"),
    ((t(4, 4096, dtype=torch.float32), t(4096, dtype=torch.float32), t(4, 4096, dtype=torch.float32)),
     "dtype must be kFloat16 or kBFloat16"),
    ((t(4, 4096), t(4096, dtype=torch.float16), t(4, 4096)), r"weight.dtype\(\) == input.dtype\(\)"),
    ((t(4, 4096), t(4096), t(4, 4096, dtype=torch.float16)), r"residual.dtype\(\) == input.dtype\(\)"),
])
def test_meta_rejects_like_the_reference(args, msg):
    with pytest.raises(RuntimeError, match=msg):
        ops.hp_rms_norm(*args, 1e-6)


def test_meta_accepts_rows_of_width_zero():
    """[..., 0] tensors hold no element: every op accepts them (view cannot
    infer their row count, so the binding counts the leading dims) and a
    width that does not match the weight is still rejected."""
    assert ops.hp_rms_norm(t(4, 0), t(0), t(4, 0), 1e-6) is None
    assert ops.hp_rms_norm(t(2, 3, 0), t(0), t(2, 3, 0), 1e-6) is None
    assert ops.relu(t(4, 0), t(4, 0)) is None
    assert ops.rms_norm(t(2, 3, 0), t(2, 3, 0), t(0), 1e-6) is None
    assert ops.fused_add_rms_norm_out(t(4, 0), t(4, 0), t(4, 0), t(0), t(4, 0), 1e-6) is None
    assert ops.hp_rms_norm_fp8(t(4, 0, dtype=torch.float8_e4m3fn), t(4, 1, dtype=torch.float32), t(4, 0), t(0),
                               t(4, 0), 1e-6) is None
    assert ops.reduce_add_rms_norm(t(4, 0), [t(4, 0), t(4, 0)], t(0), t(4, 0), 1e-6) is None
    assert ops.hp_rms_norm_mx(t(4, 0, dtype=torch.uint8), t(4, 0, dtype=torch.uint8), t(4, 0), t(0), t(4, 0), 1e-6,
                              ops.MXFP8) is None
    with pytest.raises(RuntimeError, match=r"input.size\(-1\) == hidden_dim"):
        ops.hp_rms_norm(t(4, 8), t(0), t(4, 8), 1e-6)
    with pytest.raises(RuntimeError, match="scale.numel"):
        ops.hp_rms_norm_fp8(t(4, 0, dtype=torch.float8_e4m3fn), t(3, 1, dtype=torch.float32), t(4, 0), t(0),
                            t(4, 0), 1e-6)


def test_meta_rejects_rows_that_cannot_be_flattened():
    base = t(4, 8, 256)
    x = base.transpose(0, 1)      # [8, 4, 256]: leading dims do not collapse
    with pytest.raises(RuntimeError):
        ops.hp_rms_norm(x, t(256), t(8, 4, 256), 1e-6)


def test_streamer_meta_rejects_like_the_reference():
    with pytest.raises(RuntimeError, match=r"input.dim\(\) >= 2"):
        ops.relu(t(256), t(256))
    with pytest.raises(RuntimeError, match=r"input.size\(i\) == out.size\(i\)"):
        ops.relu(t(4, 128), t(4, 256))
    with pytest.raises(RuntimeError, match="dtype must be kFloat16 or kBFloat16"):
        ops.relu(t(4, 256, dtype=torch.float32), t(4, 256, dtype=torch.float32))


def test_no_cpu_fallback():
    x = torch.zeros(4, 256, dtype=torch.bfloat16)
    w = torch.ones(256, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        ops.hp_rms_norm(x, w, x.clone(), 1e-6)
    with pytest.raises(NotImplementedError):
        ops.relu(x.clone(), x)


def test_package_points_at_in_tree_libraries():
    import os
    assert os.path.dirname(hp_rms_norm_amd.TORCH_LIB) == os.path.dirname(os.path.abspath(hp_rms_norm_amd.__file__))
    assert os.path.exists(hp_rms_norm_amd.KERNEL_LIB)


def test_fake_tensor_tracing_sees_the_mutation():
    """Alias annotations make the in-place writes visible to functionalisation."""
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        x = torch.empty(8, 512, dtype=torch.bfloat16, device=M)
        r = torch.empty(8, 512, dtype=torch.bfloat16, device=M)
        w = torch.empty(512, dtype=torch.bfloat16, device=M)
        ops.hp_rms_norm(x, w, r, 1e-6)
    schema = torch.ops.hp_rms_norm.rms_norm.default._schema
    assert [a.alias_info.is_write if a.alias_info else False for a in schema.arguments] == [True, False, True, False]


def test_fp8_op_schema_and_meta_checks():
    s = str(torch.ops.hp_rms_norm.rms_norm_fp8_quant.default._schema)
    assert s == ("hp_rms_norm::rms_norm_fp8_quant(Tensor(a!) out, Tensor(b!) scale, Tensor input, Tensor weight, "
                 "Tensor(c!) residual, float eps) -> ()")
    x, w, r = t(4, 256), t(256), t(4, 256)
    q = t(4, 256, dtype=torch.float8_e4m3fn)
    sc = torch.empty(4, 1, device=M)
    assert ops.hp_rms_norm_fp8(q, sc, x, w, r, 1e-6) is None
    with pytest.raises(RuntimeError, match="float8_e4m3fn"):
        ops.hp_rms_norm_fp8(t(4, 256), sc, x, w, r, 1e-6)
    with pytest.raises(RuntimeError, match="float32"):
        ops.hp_rms_norm_fp8(q, torch.empty(4, 1, device=M, dtype=torch.float16), x, w, r, 1e-6)
    with pytest.raises(RuntimeError, match="number of rows"):
        ops.hp_rms_norm_fp8(q, torch.empty(3, device=M), x, w, r, 1e-6)
    with pytest.raises(RuntimeError, match=r"input.size\(-1\) == hidden_dim"):
        ops.hp_rms_norm_fp8(q, sc, x, t(128), r, 1e-6)


def test_fp8_static_op_schema_and_meta_checks():
    s = str(torch.ops.hp_rms_norm.rms_norm_fp8_static_quant.default._schema)
    assert s == ("hp_rms_norm::rms_norm_fp8_static_quant(Tensor(a!) out, Tensor scale, Tensor input, Tensor weight, "
                 "Tensor(b!) residual, float eps) -> ()")
    x, w, r = t(4, 256), t(256), t(4, 256)
    q = t(4, 256, dtype=torch.float8_e4m3fn)
    sc = torch.empty(1, device=M)
    assert ops.hp_rms_norm_fp8_static(q, sc, x, w, r, 1e-6) is None
    assert ops.hp_rms_norm_fp8_static(q, torch.empty((), device=M), x, w, r, 1e-6) is None
    with pytest.raises(RuntimeError, match="float8_e4m3fn"):
        ops.hp_rms_norm_fp8_static(t(4, 256), sc, x, w, r, 1e-6)
    with pytest.raises(RuntimeError, match="float32"):
        ops.hp_rms_norm_fp8_static(q, torch.empty(1, device=M, dtype=torch.float16), x, w, r, 1e-6)
    with pytest.raises(RuntimeError, match="one element"):
        ops.hp_rms_norm_fp8_static(q, torch.empty(4, device=M), x, w, r, 1e-6)
    with pytest.raises(RuntimeError, match=r"input.size\(-1\) == hidden_dim"):
        ops.hp_rms_norm_fp8_static(q, sc, x, t(128), r, 1e-6)
    assert ops.fused_add_rms_norm_fp8_static(x, r, w, sc, 1e-6).dtype == torch.float8_e4m3fn


def test_fp8_ub_op_schema_and_meta_checks():
    s = str(torch.ops.hp_rms_norm.rms_norm_fp8_quant_ub.default._schema)
    assert s == ("hp_rms_norm::rms_norm_fp8_quant_ub(Tensor(a!) out, Tensor(b!) scale, Tensor input, "
                 "Tensor weight, Tensor(c!) residual, Tensor scale_ub, float eps) -> ()")
    x, w, r = t(4, 512), t(512), t(4, 512)
    q = t(4, 512, dtype=torch.float8_e4m3fn)
    sc, ub = torch.empty(4, 1, device=M), torch.empty(1, device=M)
    assert ops.hp_rms_norm_fp8_ub(q, sc, x, w, r, ub, 1e-6) is None
    q2, sc2 = ops.fused_add_rms_norm_fp8(t(2, 3, 512), t(2, 3, 512), w, 1e-6, scale_ub=ub)
    assert q2.shape == (2, 3, 512) and sc2.shape == (2, 3, 1)
    with pytest.raises(RuntimeError, match="scale_ub must hold one element"):
        ops.hp_rms_norm_fp8_ub(q, sc, x, w, r, torch.empty(2, device=M), 1e-6)
    with pytest.raises(RuntimeError, match="scale_ub.dtype"):
        ops.hp_rms_norm_fp8_ub(q, sc, x, w, r, torch.empty(1, device=M, dtype=torch.float16), 1e-6)


def test_fp8_group_op_schema_and_meta_checks():
    s = str(torch.ops.hp_rms_norm.rms_norm_fp8_group_quant.default._schema)
    assert s == ("hp_rms_norm::rms_norm_fp8_group_quant(Tensor(a!) out, Tensor(b!) scales, Tensor input, "
                 "Tensor weight, Tensor(c!) residual, float eps) -> ()")
    x, w, r = t(4, 512), t(512), t(4, 512)
    q = t(4, 512, dtype=torch.float8_e4m3fn)
    sc = torch.empty(4, 4, device=M)
    assert ops.hp_rms_norm_fp8_group(q, sc, x, w, r, 1e-6) is None
    q2, sc2 = ops.fused_add_rms_norm_fp8_group(t(2, 3, 512), t(2, 3, 512), w, 1e-6)
    assert q2.shape == (2, 3, 512) and q2.dtype == torch.float8_e4m3fn and sc2.shape == (2, 3, 4)
    assert sc2.dtype == torch.float32
    with pytest.raises(RuntimeError, match="128"):
        ops.hp_rms_norm_fp8_group(t(4, 320, dtype=torch.float8_e4m3fn), torch.empty(4, 2, device=M), t(4, 320),
                                  t(320), t(4, 320), 1e-6)
    with pytest.raises(RuntimeError, match="float8_e4m3fn"):
        ops.hp_rms_norm_fp8_group(t(4, 512), sc, x, w, r, 1e-6)
    with pytest.raises(RuntimeError, match="float32"):
        ops.hp_rms_norm_fp8_group(q, torch.empty(4, 4, device=M, dtype=torch.float16), x, w, r, 1e-6)
    with pytest.raises(RuntimeError, match="hidden / 128"):
        ops.hp_rms_norm_fp8_group(q, torch.empty(4, 16, device=M), x, w, r, 1e-6)
    # column-major scales (a transposed view) pass the checks; scales that overlap themselves do not
    assert ops.hp_rms_norm_fp8_group(q, torch.empty(4, 4, device=M).t(), x, w, r, 1e-6) is None
    q3, sc3 = ops.fused_add_rms_norm_fp8_group(t(2, 3, 512), t(2, 3, 512), w, 1e-6, column_major_scales=True,
                                               scale_row_align=4)
    assert sc3.shape == (2, 3, 4) and sc3.stride() == (3, 1, 8)
    with pytest.raises(RuntimeError, match="overlap themselves"):
        ops.hp_rms_norm_fp8_group(q, torch.empty(1, 4, device=M).expand(4, 4), x, w, r, 1e-6)


def test_out_of_place_and_reduce_schemas():
    s = str(torch.ops.hp_rms_norm.rms_norm_out.default._schema)
    assert s == ("hp_rms_norm::rms_norm_out(Tensor(a!) out, Tensor(b!) residual_out, Tensor input, Tensor weight, "
                 "Tensor residual, float eps) -> ()")
    s = str(torch.ops.hp_rms_norm.reduce_add_rms_norm.default._schema)
    assert s == ("hp_rms_norm::reduce_add_rms_norm(Tensor(a!) out, Tensor[] parts, Tensor weight, "
                 "Tensor(b!) residual, float eps) -> ()")


def test_out_of_place_meta_checks():
    x, r, w = t(4, 256), t(4, 256), t(256)
    assert ops.fused_add_rms_norm_out(t(4, 256), t(4, 256), x, w, r, 1e-6) is None
    assert ops.fused_add_rms_norm_out(x, r, x, w, r, 1e-6) is None          # in place is allowed
    out, res = ops.fused_add_rms_norm(x, r, w, 1e-6)
    assert out.shape == x.shape and res.shape == r.shape and out.device.type == M
    with pytest.raises(RuntimeError, match=r"input.size\(-1\) == hidden_dim"):
        ops.fused_add_rms_norm_out(t(4, 256), t(4, 256), x, t(128), r, 1e-6)
    with pytest.raises(RuntimeError, match="dtype"):
        ops.fused_add_rms_norm_out(t(4, 256, dtype=torch.float16), t(4, 256), x, w, r, 1e-6)
    with pytest.raises(RuntimeError, match=r"input.size\(i\) == residual.size\(i\)"):
        ops.fused_add_rms_norm_out(t(4, 256), t(5, 256), x, w, r, 1e-6)


def test_reduce_meta_checks():
    r, w = t(4, 256), t(256)
    parts = [t(4, 256) for _ in range(3)]
    assert ops.reduce_add_rms_norm(t(4, 256), parts, w, r, 1e-6) is None
    assert ops.reduce_add_rms_norm(parts[0], parts, w, r, 1e-6) is None     # out may be a part
    with pytest.raises(RuntimeError, match="1 to 8"):
        ops.reduce_add_rms_norm(t(4, 256), [], w, r, 1e-6)
    with pytest.raises(RuntimeError, match="1 to 8"):
        ops.reduce_add_rms_norm(t(4, 256), [t(4, 256) for _ in range(9)], w, r, 1e-6)
    with pytest.raises(RuntimeError, match="shape"):
        ops.reduce_add_rms_norm(t(4, 256), [t(4, 256), t(2, 256)], w, r, 1e-6)
    with pytest.raises(RuntimeError, match="dtype"):
        ops.reduce_add_rms_norm(t(4, 256), [t(4, 256), t(4, 256, dtype=torch.float16)], w, r, 1e-6)
    with pytest.raises(RuntimeError, match="one row stride"):
        ops.reduce_add_rms_norm(t(4, 256), [t(4, 256), t(4, 512)[:, :256]], w, r, 1e-6)


def test_mx_op_schema_and_meta_checks():
    s = str(torch.ops.hp_rms_norm.rms_norm_mx_quant.default._schema)
    assert s == ("hp_rms_norm::rms_norm_mx_quant(Tensor(a!) out, Tensor(b!) scales, Tensor input, Tensor weight, "
                 "Tensor(c!) residual, int format, float eps) -> ()")
    x, w, r = t(4, 256), t(256), t(4, 256)
    q4, sc = ops.fused_add_rms_norm_mxfp4(x, r, w, 1e-6)
    assert q4.shape == (4, 128) and q4.dtype == torch.float4_e2m1fn_x2
    assert sc.shape == (4, 8) and sc.dtype == torch.float8_e8m0fnu
    q8, sc = ops.fused_add_rms_norm_mxfp8(x, r, w, 1e-6)
    assert q8.shape == (4, 256) and q8.dtype == torch.float8_e4m3fn
    u8 = lambda *sh: torch.empty(*sh, dtype=torch.uint8, device=M)   # noqa: E731
    assert ops.hp_rms_norm_mx(u8(4, 128), u8(4, 8), x, w, r, 1e-6, ops.MXFP4) is None
    with pytest.raises(RuntimeError, match="32"):
        ops.hp_rms_norm_mx(u8(4, 120), u8(4, 7), t(4, 240), t(240), t(4, 240), 1e-6, ops.MXFP4)
    with pytest.raises(RuntimeError, match="hidden / 2"):
        ops.hp_rms_norm_mx(u8(4, 256), u8(4, 8), x, w, r, 1e-6, ops.MXFP4)
    with pytest.raises(RuntimeError, match="hidden / 32"):
        ops.hp_rms_norm_mx(u8(4, 128), u8(4, 4), x, w, r, 1e-6, ops.MXFP4)
    with pytest.raises(RuntimeError, match="format"):
        ops.hp_rms_norm_mx(u8(4, 128), u8(4, 8), x, w, r, 1e-6, 3)
    with pytest.raises(RuntimeError, match="float8_e4m3fn or uint8"):
        ops.hp_rms_norm_mx(t(4, 256), u8(4, 8), x, w, r, 1e-6, ops.MXFP8)


def test_missing_native_library_is_an_import_error(tmp_path):
    """The package has no fallback: a copy of it without its built libraries
    refuses to import, naming the build command."""
    import shutil
    import subprocess
    import sys
    pkg = tmp_path / "hp_rms_norm_amd"
    src = os.path.dirname(os.path.abspath(hp_rms_norm_amd.__file__))
    shutil.copytree(src, pkg, ignore=shutil.ignore_patterns("*.so", "__pycache__", "csrc"))
    code = "import hp_rms_norm_amd"
    p = subprocess.run([sys.executable, "-c", code], cwd=tmp_path, capture_output=True, text=True, timeout=300)
    assert p.returncode != 0
    assert "ImportError" in p.stderr and "not built" in p.stderr and "hp_rms_norm_amd/build.py" in p.stderr


def test_fp8_meta_rejects_overlapping_outputs():
    """The FP8 rows and the scales are written while input and residual are
    read: any overlap among them is refused."""
    x, w, r = t(4, 256), t(256), t(4, 256)
    qbuf = torch.empty(4 * 256 + 64, dtype=torch.uint8, device=M)
    q = qbuf[:1024].view(torch.float8_e4m3fn).view(4, 256)
    sc = torch.empty(4, 1, device=M)
    assert ops.hp_rms_norm_fp8(q, sc, x, w, r, 1e-6) is None
    rbuf = torch.empty(4 * 256 * 2, dtype=torch.uint8, device=M)
    r_shared = rbuf.view(torch.bfloat16).view(4, 256)
    xbuf = torch.empty(4 * 256 * 2, dtype=torch.uint8, device=M)
    x_shared = xbuf.view(torch.bfloat16).view(4, 256)
    cases = [
        (rbuf[:1024].view(torch.float8_e4m3fn).view(4, 256), sc, x, r_shared),      # out on residual
        (xbuf[:1024].view(torch.float8_e4m3fn).view(4, 256), sc, x_shared, r),      # out on input
        (q, rbuf[:16].view(torch.float32).view(4, 1), x, r_shared),                  # scale on residual
        (q, xbuf[:16].view(torch.float32).view(4, 1), x_shared, r),                  # scale on input
        (q, qbuf[:16].view(torch.float32).view(4, 1), x, r),                         # scale on out
    ]
    for out, scale, inp, res in cases:
        with pytest.raises(RuntimeError, match="written-to"):
            ops.hp_rms_norm_fp8(out, scale, inp, w, res, 1e-6)


def test_mx_meta_rejects_outputs_on_the_input():
    w, r = t(256), t(4, 256)
    xbuf = torch.empty(4 * 256 * 2, dtype=torch.uint8, device=M)
    x_shared = xbuf.view(torch.bfloat16).view(4, 256)
    u8 = lambda *sh: torch.empty(*sh, dtype=torch.uint8, device=M)   # noqa: E731
    with pytest.raises(RuntimeError, match="written-to"):
        ops.hp_rms_norm_mx(xbuf[:512].view(4, 128), u8(4, 8), x_shared, w, r, 1e-6, ops.MXFP4)
    with pytest.raises(RuntimeError, match="written-to"):
        ops.hp_rms_norm_mx(u8(4, 128), xbuf[:32].view(4, 8), x_shared, w, r, 1e-6, ops.MXFP4)
