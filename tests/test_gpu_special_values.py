"""GPU parity on rows of special values (tests/helpers.py, SPECIAL_PATTERNS):
NaN, infinities, zero rows with eps = 0, binary32 overflow of a square and of
the sum of squares, subnormals and negative zeros, against the CPU oracle,
whose handling of each is pinned against the reference's torch formula
(tests/test_oracle.py, pin_special_values).

Bar: as everywhere, the residual bit-exact and the output within 1 ulp (and
atol = rtol = 1e-2), NaN exactly where the oracle has NaN.  NaN bit patterns
are not compared: IEEE 754 leaves them open, and torch's own differ between
its vectorised and scalar code.
"""
import pytest
import torch

from helpers import (DT, assert_output_close, assert_residual_exact, bits, oracle_fused, special_inputs,
                     special_weight)
from oracle import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

# (rows, hidden, row stride - hidden): one shape per kind of kernel the in-place
# dispatch runs, with the kernel it picks on 256 CUs
FUSED_CASES = [
    (28, 1024, 0),       # latency rows (64 x 2)
    (2048, 1024, 0),     # 32 x 4, eight rows per workgroup
    (2560, 2048, 0),     # wide rows (32 x 8, two rows per one-wave workgroup)
    (1024, 4096, 0),     # one-wave rows (64 x 8)
    (4096, 4096, 0),     # 256 x 2, runs of 32 row groups per XCD
    (1024, 6144, 0),     # two-wave rows (128 x 6)
    (2048, 8192, 0),     # 512 x 2, runs of 64 row groups per XCD
    (1024, 12288, 0),    # 512 x 3
    (600, 16384, 0),     # the LDS tier, 256 x 8 (4)
    (300, 32768, 0),     # 1024 x 4
    (300, 65536, 0),     # 1024 x 8 (4)
    (1200, 8192, 8),     # rows 16 bytes off the 128-byte grid: the rotated variant
    (1024, 8192, 1),     # rows 2 bytes apart in phase: shifted rows, the weight staged in LDS
    (1024, 4097, 0),     # odd width: the tail variant
    (16, 70000, 0),      # past the vector tiers: the general kernel
]


@pytest.fixture(scope="module")
def abi():
    assert torch.cuda.is_available(), "the gpu tests need a HIP device"
    import hp_rms_norm_amd  # noqa: F401  (registers the torch ops; fails loudly if unbuilt)
    from hp_rms_norm_amd import abi as a
    a.lib()
    return a


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _on_device(t, pad):
    """`t` copied to the GPU as rows of a [rows, hidden + pad] buffer."""
    rows, hidden = t.shape
    buf = torch.zeros(rows, hidden + pad, dtype=t.dtype, device=DEV)
    view = buf[:, :hidden]
    view.copy_(t)
    return view


@pytest.mark.parametrize("eps", [0.0, 1e-6], ids=["eps0", "eps1e-6"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_fused_special_values(abi, dtype, eps):
    for rows, hidden, pad in FUSED_CASES:
        tag = f"special {rows}x{hidden}+{pad} {dtype} eps {eps}"
        print(tag, flush=True)
        x, r, w = special_inputs(rows, hidden, dtype, seed=rows + hidden)
        want_out, want_res = oracle_fused(x, r, w, eps, dtype)
        xd, rd, wd = _on_device(x, pad), _on_device(r, pad), w.to(DEV)
        abi.fused_add_rmsnorm(xd.data_ptr(), wd.data_ptr(), rd.data_ptr(), rows, hidden, xd.stride(0),
                              rd.stride(0), DT[dtype], eps, _stream())
        torch.cuda.synchronize()
        assert_residual_exact(bits(rd), want_res, dtype, "residual " + tag)
        assert_output_close(bits(xd), want_out, dtype, "output " + tag)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_fused_special_weight(abi, dtype):
    """The same rows with a weight of special values (helpers.special_weight):
    zeros, infinities, a NaN, a subnormal and the largest magnitudes."""
    for rows, hidden, pad in FUSED_CASES:
        tag = f"special weight {rows}x{hidden}+{pad} {dtype}"
        print(tag, flush=True)
        x, r, w = special_inputs(rows, hidden, dtype, seed=rows + 2 * hidden)
        w = special_weight(w)
        want_out, want_res = oracle_fused(x, r, w, 1e-6, dtype)
        xd, rd, wd = _on_device(x, pad), _on_device(r, pad), w.to(DEV)
        abi.fused_add_rmsnorm(xd.data_ptr(), wd.data_ptr(), rd.data_ptr(), rows, hidden, xd.stride(0),
                              rd.stride(0), DT[dtype], 1e-6, _stream())
        torch.cuda.synchronize()
        assert_residual_exact(bits(rd), want_res, dtype, "residual " + tag)
        assert_output_close(bits(xd), want_out, dtype, "output " + tag)


@pytest.mark.parametrize("eps", [0.0, 1e-6], ids=["eps0", "eps1e-6"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_other_forms_special_values(abi, dtype, eps):
    """Plain RMSNorm, the out-of-place op and the partial-sum form (parts x and
    r, residual 0) on the same rows, each against its oracle."""
    for rows, hidden in ((28, 4096), (1024, 4096), (600, 16384), (300, 32768)):
        tag = f"special {rows}x{hidden} {dtype} eps {eps}"
        print(tag, flush=True)
        x, r, w = special_inputs(rows, hidden, dtype, seed=rows * 3 + hidden)
        xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
        code = DT[dtype]
        # plain RMSNorm of x
        od = torch.empty_like(xd)
        abi.rmsnorm(od.data_ptr(), xd.data_ptr(), wd.data_ptr(), rows, hidden, hidden, hidden, code, eps, _stream())
        torch.cuda.synchronize()
        assert_output_close(bits(od), oracle.rmsnorm(bits(x), bits(w), eps, code, threads=8), dtype,
                            "plain " + tag)
        # out of place: input and residual untouched
        od, rod = torch.empty_like(xd), torch.empty_like(rd)
        abi.fused_add_rmsnorm_out(od.data_ptr(), rod.data_ptr(), xd.data_ptr(), rd.data_ptr(), wd.data_ptr(),
                                  rows, hidden, hidden, hidden, hidden, hidden, code, eps, _stream())
        torch.cuda.synchronize()
        want_out, want_res = oracle_fused(x, r, w, eps, dtype)
        assert_residual_exact(bits(rod), want_res, dtype, "out-of-place residual " + tag)
        assert_output_close(bits(od), want_out, dtype, "out-of-place output " + tag)
        assert_residual_exact(bits(xd), bits(x), dtype, "out-of-place input untouched " + tag)
        # partial sums: a = rne(x + r), then the fused op with a zero residual
        zero = torch.zeros_like(rd)
        od = torch.empty_like(xd)
        abi.reduce_add_rmsnorm(od.data_ptr(), [xd.data_ptr(), rd.data_ptr()], wd.data_ptr(), zero.data_ptr(),
                               rows, hidden, hidden, hidden, hidden, code, eps, _stream())
        torch.cuda.synchronize()
        want_out, want_res = oracle.reduce_add_rmsnorm([bits(x), bits(r)], bits(w), bits(torch.zeros_like(r)), eps,
                                                       code, threads=8)
        assert_residual_exact(bits(zero), want_res, dtype, "partial-sum residual " + tag)
        assert_output_close(bits(od), want_out, dtype, "partial-sum output " + tag)


# eps that swamps the mean square (1, 1e30) or overflows binary32 (1e39, inf):
# the output goes to zero, NaN where a factor is infinite
LARGE_EPS = [1.0, 1e30, 1e39, float("inf")]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_large_eps(abi, dtype):
    """The fused op on the special rows with eps past the mean square, up to
    infinity, at one shape per kernel kind of the table, the tail variant and
    the general kernel, and plain RMSNorm at two widths."""
    code = DT[dtype]
    for rows, hidden, pad in [c for c in FUSED_CASES if c[1] in (1024, 4096, 16384, 32768, 4097, 70000)]:
        x, r, w = special_inputs(rows, hidden, dtype, seed=rows + 3 * hidden)
        for eps in LARGE_EPS:
            tag = f"large eps {rows}x{hidden}+{pad} {dtype} eps {eps}"
            print(tag, flush=True)
            want_out, want_res = oracle_fused(x, r, w, eps, dtype)
            xd, rd, wd = _on_device(x, pad), _on_device(r, pad), w.to(DEV)
            abi.fused_add_rmsnorm(xd.data_ptr(), wd.data_ptr(), rd.data_ptr(), rows, hidden, xd.stride(0),
                                  rd.stride(0), code, eps, _stream())
            torch.cuda.synchronize()
            assert_residual_exact(bits(rd), want_res, dtype, "residual " + tag)
            assert_output_close(bits(xd), want_out, dtype, "output " + tag)
    for rows, hidden in ((28, 4096), (300, 32768)):
        x, _, w = special_inputs(rows, hidden, dtype, seed=rows + hidden)
        xd, wd = x.to(DEV), w.to(DEV)
        for eps in LARGE_EPS:
            od = torch.empty_like(xd)
            abi.rmsnorm(od.data_ptr(), xd.data_ptr(), wd.data_ptr(), rows, hidden, hidden, hidden, code, eps,
                        _stream())
            torch.cuda.synchronize()
            assert_output_close(bits(od), oracle.rmsnorm(bits(x), bits(w), eps, code, threads=8), dtype,
                                f"plain large eps {rows}x{hidden} {dtype} eps {eps}")
