"""GPU parity of the fused add+RMSNorm with an FP8 (OCP e4m3fn) output and one
given scale for every row (static per-tensor quantisation).

Pins: the residual is bit-exact against the oracle; q equals, bit for bit,
torch's static quantisation (e4m3fn(clamp(y * reciprocal(scale), +-448))) of
the 16-bit output the same kernel family produces for the same inputs (the
16-bit op run with the FP8 table's lane mapping); against the CPU oracle q is
the quantisation of a y within one 16-bit ulp of the oracle's output.
`input` and the scale are not modified.  NaN encodings differ (hardware 0xFF,
torch 0x7F): NaN compares equal to NaN here.
"""
import numpy as np
import pytest
import torch

from helpers import (DT, assert_fp8_from_y_within_one_ulp, assert_residual_exact, bits, from_bits, lane_mapping,
                     make_inputs, special_inputs)
from oracle import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def ops():
    assert torch.cuda.is_available(), "the gpu tests need a HIP device"
    import hp_rms_norm_amd
    return hp_rms_norm_amd


def torch_quantise_static(y, scale):
    yf = y.detach().cpu().float()
    q = (yf * torch.reciprocal(torch.tensor(scale, dtype=torch.float32))).clamp(-448.0, 448.0)
    return q.to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def q_bits(q):
    return q.detach().cpu().contiguous().view(torch.uint8).numpy()


def run_case(ops, rows, hidden, dtype, seed, scale, dist="bench", eps=1e-6, special=False):
    from hp_rms_norm_amd import abi
    if special:
        x, r, w = special_inputs(rows, hidden, dtype, seed)
    else:
        x, r, w = make_inputs(rows, hidden, dtype, seed, dist)
    xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
    sd = torch.tensor([scale], dtype=torch.float32, device=DEV)
    q = ops.fused_add_rms_norm_fp8_static(xd, rd, wd, sd, eps)
    # the same inputs through the 16-bit op with the FP8 kernel's lane mapping
    # (the same fp32 reduction order, hence the same y)
    cfg = lane_mapping(abi, abi.select_config(rows, hidden, DT[dtype], abi.MODE_FP8))
    y, r16 = x.to(DEV), r.to(DEV)
    abi.BENCH.fused_add_rmsnorm(y.data_ptr(), wd.data_ptr(), r16.data_ptr(), rows, hidden, hidden, hidden, DT[dtype],
                                eps, torch.cuda.current_stream().cuda_stream, None if cfg.tier == 3 else cfg)
    torch.cuda.synchronize()
    tag = f"{rows}x{hidden} {dtype} seed {seed} scale {scale}"
    assert torch.equal(xd.cpu().view(torch.int16), x.view(torch.int16)), "input modified " + tag
    assert torch.equal(sd.cpu().view(torch.int32), torch.tensor([scale], dtype=torch.float32).view(torch.int32)), \
        "scale modified " + tag
    assert torch.equal(rd.view(torch.int16), r16.view(torch.int16)), "residual differs from the 16-bit op " + tag
    d = oracle.e4m3_ulp_distance(q_bits(q), torch_quantise_static(y, scale))
    assert d.max() == 0, f"q differs from torch's quantisation of y: {tag}"
    oy, ores = oracle.fused_add_rmsnorm(bits(x), bits(w), bits(r), eps, DT[dtype],
                                        threads=min(16, oracle.max_threads()))
    assert_residual_exact(bits(rd), ores, dtype, "residual " + tag)
    with np.errstate(divide="ignore", over="ignore"):
        isc = np.float32(1.0) / np.float32(scale)
    assert_fp8_from_y_within_one_ulp(q_bits(q), oy, isc, dtype, "q " + tag)


def test_fp8_static_golden_through_torch_op(ops, golden):
    """torch's static quantisation of torch's own 16-bit output (golden
    vectors): the residual bit-exact, q the quantisation of a y within one
    16-bit ulp of torch's output."""
    n = 0
    for name, c in golden.items():
        if c["kind"] != "fp8_static":
            continue
        dtype = torch.bfloat16 if c["dtype"] == "bf16" else torch.float16
        x, r, w = (from_bits(c[k], dtype).to(DEV) for k in ("x", "r", "w"))
        q = ops.fused_add_rms_norm_fp8_static(x, r, w, torch.tensor([c["scale"]], device=DEV), c["eps"])
        torch.cuda.synchronize()
        assert_residual_exact(bits(r), c["res"], dtype, name)
        assert_fp8_from_y_within_one_ulp(q_bits(q), c["out"], np.float32(1.0) / np.float32(c["scale"]), dtype, name)
        n += 1
    assert n >= 2


@pytest.mark.parametrize("rows,hidden,dtype", [
    (4096, 4096, torch.bfloat16), (4096, 8192, torch.bfloat16), (4096, 16384, torch.bfloat16),
    (4096, 32768, torch.bfloat16), (4096, 5120, torch.float16), (4096, 7168, torch.float16),
    (1, 4096, torch.bfloat16), (32, 8192, torch.bfloat16), (512, 4096, torch.bfloat16)],
    ids=lambda v: str(v).replace("torch.", ""))
def test_fp8_static_baseline_shapes(ops, rows, hidden, dtype):
    print("fp8 static case", rows, hidden, dtype, flush=True)
    # a scale that sends the largest outputs past 448 (clamped) and one that does not
    for scale in (0.01, 0.05):
        run_case(ops, rows, hidden, dtype, seed=rows + hidden, scale=scale,
                 dist="outliers" if rows <= 512 else "bench")


def test_fp8_static_every_table_entry(ops):
    """H at every breakpoint of the FP8 table (and one below), with 1100 rows
    (the bandwidth rows) and 7 rows (the latency rows), and past the vector
    tiers (the general kernels)."""
    for hidden in (128, 256, 512, 1024, 1032, 2048, 3072, 4096, 4104, 5120, 8192, 12288, 16384, 24576, 32768, 65536,
                   520, 4088, 70000):
        for rows in (1100, 7):
            if hidden == 70000 and rows == 1100:
                continue
            print("fp8 static table", rows, hidden, flush=True)
            run_case(ops, rows, hidden, torch.bfloat16, seed=hidden + rows, scale=0.02)


@pytest.mark.parametrize("hidden", [1, 13, 255, 1001, 4097, 9999, 16385])
def test_fp8_static_odd_widths(ops, hidden):
    run_case(ops, 37, hidden, torch.bfloat16, seed=hidden, scale=0.03)
    run_case(ops, 5, hidden, torch.float16, seed=hidden + 1, scale=0.03)


def test_fp8_static_special_rows_and_scales(ops):
    """Rows of special values (NaN, infinities, zero rows, overflow of the sum
    of squares, subnormals), and scales that are subnormal, huge, zero,
    infinite and NaN: every element as torch's static quantisation of y."""
    for rows, hidden in ((28, 1024), (300, 4096), (40, 32768), (16, 70000)):
        for scale in (0.02, 1.0, 2.0 ** -140, 1e30, 0.0, float("inf"), float("nan")):
            print("fp8 static special", rows, hidden, scale, flush=True)
            run_case(ops, rows, hidden, torch.bfloat16, seed=rows + hidden, scale=scale, special=True)


def test_fp8_static_strided_misaligned_output(ops):
    from hp_rms_norm_amd import abi
    rows, hidden, eps, dtype, scale = 40, 2048, 1e-6, torch.bfloat16, 0.02
    x, r, w = make_inputs(rows, hidden, dtype, 78)
    oy, ores = oracle.fused_add_rmsnorm(bits(x), bits(w), bits(r), eps, oracle.BF16)
    for offset, pad in ((0, 64), (1, 3)):
        xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
        sd = torch.tensor([scale], dtype=torch.float32, device=DEV)
        buf = torch.zeros(rows, hidden + pad + offset, dtype=torch.uint8, device=DEV)
        qv = buf[:, offset:offset + hidden]
        abi.fused_add_rmsnorm_fp8_static(qv.data_ptr(), sd.data_ptr(), xd.data_ptr(), wd.data_ptr(), rd.data_ptr(),
                                         rows, hidden, qv.stride(0), hidden, hidden, abi.DTYPE_BF16, eps,
                                         torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert_residual_exact(bits(rd), ores, dtype)
        assert_fp8_from_y_within_one_ulp(qv.cpu().numpy(), oy, np.float32(1.0) / np.float32(scale), dtype)
        assert not buf[:, :offset].any() and not buf[:, offset + hidden:].any()


def test_fp8_static_equals_dynamic_with_the_same_scales(ops):
    """Where every row's dynamic scale is the same number, the static form with
    that number gives the dynamic form's q bit for bit (rows that are copies
    of one row, in place, so both forms run the same kernel shapes)."""
    rows, hidden = 64, 4096
    x, r, w = make_inputs(1, hidden, torch.bfloat16, 5)
    x, r = x.repeat(rows, 1), r.repeat(rows, 1)
    xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
    q_dyn, sc = ops.fused_add_rms_norm_fp8(xd, rd, wd, 1e-6)
    torch.cuda.synchronize()
    assert torch.unique(sc).numel() == 1
    xd2, rd2 = x.to(DEV), r.to(DEV)
    q_st = ops.fused_add_rms_norm_fp8_static(xd2, rd2, wd, sc[:1].reshape(1).clone(), 1e-6)
    torch.cuda.synchronize()
    assert np.array_equal(q_bits(q_st), q_bits(q_dyn))
    assert torch.equal(rd2.view(torch.int16), rd.view(torch.int16))
