"""GPU parity of the fused add+RMSNorm with FP8 (OCP e4m3fn) per-row output.

Pins: the residual is bit-exact against the oracle; q and scale equal, bit
for bit, torch's quantisation of the 16-bit output the same kernel family
produces for the same inputs (the bf16 op run on a copy); against the CPU
oracle q is the quantisation of a y within one 16-bit ulp of the oracle's
output, and scale that of an amax within one ulp of the oracle's (golden
vectors: within one FP8 step).
`input` is not modified.  NaN encodings differ (hardware 0xFF, torch 0x7F):
NaN compares equal to NaN here.
"""
import numpy as np
import pytest
import torch

from helpers import (DT, assert_fp8_from_y_within_one_ulp, assert_group_scales, assert_residual_exact, bits, from_bits,
                     lane_mapping, make_inputs)
from oracle import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def ops():
    assert torch.cuda.is_available(), "the gpu tests need a HIP device"
    import hp_rms_norm_amd
    return hp_rms_norm_amd


def torch_quantise(y):
    # on the CPU: ATen's HIP kernels turn division by a scalar into a
    # multiplication by its reciprocal, the CPU path divides
    yf = y.detach().cpu().float()
    scale = torch.clamp(yf.abs().amax(-1, keepdim=True) / 448.0, min=torch.finfo(torch.float32).tiny)
    q = (yf * (1.0 / scale)).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q, scale


def q_bits(q):
    return q.detach().cpu().contiguous().view(torch.uint8).numpy()


def run_case(ops, rows, hidden, dtype, seed, dist="bench", eps=1e-6):
    x, r, w = make_inputs(rows, hidden, dtype, seed, dist)
    xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
    q, sc = ops.fused_add_rms_norm_fp8(xd, rd, wd, eps)
    # the same inputs through the 16-bit op with the FP8 kernel's lane mapping
    # (the same fp32 reduction order, hence the same y); the bench library
    # holds that shape for the 16-bit op where the FP8 table has a row of its own
    from hp_rms_norm_amd import abi
    cfg = lane_mapping(abi, abi.select_config(rows, hidden, DT[dtype], 2))
    y, r16 = x.to(DEV), r.to(DEV)
    abi.BENCH.fused_add_rmsnorm(y.data_ptr(), wd.data_ptr(), r16.data_ptr(), rows, hidden, hidden, hidden, DT[dtype],
                                eps, torch.cuda.current_stream().cuda_stream, None if cfg.tier == 3 else cfg)
    torch.cuda.synchronize()
    tag = f"{rows}x{hidden} {dtype} seed {seed}"
    assert torch.equal(xd.cpu().view(torch.int16), x.view(torch.int16)), "input modified " + tag
    assert torch.equal(rd.view(torch.int16), r16.view(torch.int16)), "residual differs from the 16-bit op " + tag
    tq, tsc = torch_quantise(y)
    sc_c, tsc_c = sc.reshape(-1).cpu(), tsc.reshape(-1)
    assert torch.equal(sc_c.view(torch.int32), tsc_c.view(torch.int32)) or \
        torch.allclose(sc_c, tsc_c, rtol=0, atol=0, equal_nan=True), "scale " + tag
    d = oracle.e4m3_ulp_distance(q_bits(q), q_bits(tq))
    assert d.max() == 0, f"q differs from torch's quantisation of y: {tag}"
    # against the CPU oracle: the quantisation of a y within one 16-bit ulp of its output
    oy, ores = oracle.fused_add_rmsnorm(bits(x), bits(w), bits(r), eps, DT[dtype],
                                        threads=min(16, oracle.max_threads()))
    assert_residual_exact(bits(rd), ores, dtype, "residual " + tag)
    scales = sc.reshape(-1, 1).cpu().numpy()
    assert_group_scales(scales, oy, hidden, dtype, "scale " + tag)
    with np.errstate(divide="ignore"):
        assert_fp8_from_y_within_one_ulp(q_bits(q), oy, np.float32(1.0) / scales, dtype, "q " + tag)
    return q, sc


def test_fp8_golden_through_torch_op(ops, golden):
    for name, c in golden.items():
        if c["kind"] != "fp8":
            continue
        dtype = torch.bfloat16 if c["dtype"] == "bf16" else torch.float16
        x, r, w = (from_bits(c[k], dtype).to(DEV) for k in ("x", "r", "w"))
        q, sc = ops.fused_add_rms_norm_fp8(x, r, w, c["eps"])
        torch.cuda.synchronize()
        assert_residual_exact(bits(r), c["res"], dtype, name)
        d = oracle.e4m3_ulp_distance(q_bits(q), c["q"])
        assert d.max() <= 1 and (d != 0).mean() < 1e-3, name
        np.testing.assert_allclose(sc.reshape(-1).cpu().numpy(), c["scale"], rtol=2.0 ** -7, equal_nan=True)


@pytest.mark.parametrize("rows,hidden,dtype", [
    (4096, 4096, torch.bfloat16), (4096, 8192, torch.bfloat16), (4096, 16384, torch.bfloat16),
    (4096, 32768, torch.bfloat16), (4096, 5120, torch.float16), (4096, 7168, torch.float16),
    (1, 4096, torch.bfloat16), (32, 8192, torch.bfloat16), (512, 4096, torch.bfloat16)],
    ids=lambda v: str(v).replace("torch.", ""))
def test_fp8_baseline_shapes(ops, rows, hidden, dtype):
    print("fp8 case", rows, hidden, dtype, flush=True)
    run_case(ops, rows, hidden, dtype, seed=rows + hidden, dist="outliers" if rows <= 512 else "bench")


def test_fp8_every_table_entry(ops):
    """H at every breakpoint of the table (and one below), with 1100 rows (the
    bandwidth rows) and 7 rows (the latency rows)."""
    for hidden in (128, 256, 512, 1024, 1032, 2048, 3072, 4096, 4104, 5120, 8192, 12288, 16384, 24576, 32768, 65536,
                   520, 4088):
        for rows in (1100, 7):
            print("fp8 table", rows, hidden, flush=True)
            run_case(ops, rows, hidden, torch.bfloat16, seed=hidden + rows)


# odd widths: the tail variants from 8 up, the general tier below
@pytest.mark.parametrize("hidden", [1, 13, 255, 700, 1001, 2049, 4097, 7167, 9999, 13313, 16383, 16385])
def test_fp8_odd_widths(ops, hidden):
    run_case(ops, 37, hidden, torch.bfloat16, seed=hidden)
    run_case(ops, 5, hidden, torch.float16, seed=hidden + 1)


def test_fp8_strided_misaligned_output_and_special_rows(ops):
    from hp_rms_norm_amd import abi
    rows, hidden, eps, dtype = 40, 2048, 1e-6, torch.bfloat16
    x, r, w = make_inputs(rows, hidden, dtype, 77)
    x[0].zero_()
    r[0].zero_()
    x[1, 5] = float("nan")
    oq, osc, ores = oracle.fused_add_rmsnorm_fp8(bits(x), bits(w), bits(r), eps, oracle.BF16)
    assert osc[0] == np.finfo(np.float32).tiny and np.isnan(osc[1])
    for offset, pad in ((0, 64), (1, 3)):
        xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
        buf = torch.zeros(rows, hidden + pad + offset, dtype=torch.uint8, device=DEV)
        qv = buf[:, offset:offset + hidden]
        sc = torch.full((rows,), 7.0, device=DEV)
        abi.fused_add_rmsnorm_fp8(qv.data_ptr(), sc.data_ptr(), xd.data_ptr(), wd.data_ptr(), rd.data_ptr(), rows,
                                  hidden, qv.stride(0), hidden, hidden, abi.DTYPE_BF16, eps,
                                  torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert_residual_exact(bits(rd), ores, dtype)
        oy, _ = oracle.fused_add_rmsnorm(bits(x), bits(w), bits(r), eps, oracle.BF16)
        scales = sc.reshape(-1, 1).cpu().numpy()
        assert_group_scales(scales, oy, hidden, dtype)
        with np.errstate(divide="ignore"):
            assert_fp8_from_y_within_one_ulp(qv.cpu().numpy(), oy, np.float32(1.0) / scales, dtype)
        assert not buf[:, :offset].any() and not buf[:, offset + hidden:].any()
        assert not qv[0].any()                                   # zero row -> zero codes
        assert ((qv[1].cpu().numpy() & 0x7F) == 0x7F).all()       # NaN row -> NaN codes


def test_fp8_bytes_move_less(ops):
    """FP8 output: the op writes H bytes per row instead of 2H, and still
    updates the residual; checks the written sizes through the returned tensors."""
    x, r, w = (t.to(DEV) for t in make_inputs(8, 4096, torch.bfloat16, 3))
    q, sc = ops.fused_add_rms_norm_fp8(x, r, w, 1e-6)
    assert q.dtype == torch.float8_e4m3fn and q.shape == x.shape and q.element_size() == 1
    assert sc.shape == (8, 1) and sc.dtype == torch.float32
