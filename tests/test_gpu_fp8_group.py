"""GPU parity of the fused add+RMSNorm with an FP8 (OCP e4m3fn) output and one
float32 scale per 128 consecutive elements of a row (per-token-group
quantisation, 1 x 128 groups).

Pins: the residual is bit-exact against the oracle; q and the scales equal,
bit for bit, torch's per-group quantisation of the 16-bit output the same
kernel family produces for the same inputs (the 16-bit op run with this
form's lane mapping); against the CPU oracle q is the quantisation of a y
within one 16-bit ulp of the oracle's output and the scales those of a group
maximum within one ulp of the oracle's (one ulp of a subnormal y is a factor
of two, so no fixed FP8 step bound holds there).  `input` is not modified.
NaN encodings differ (hardware 0xFF, torch 0x7F): NaN compares equal to NaN.
"""
import numpy as np
import pytest
import torch

from helpers import (DT, assert_fp8_from_y_within_one_ulp, assert_group_scales, assert_residual_exact, bits, from_bits,
                     lane_mapping, make_inputs, special_inputs)
from oracle import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def ops():
    assert torch.cuda.is_available(), "the gpu tests need a HIP device"
    import hp_rms_norm_amd
    return hp_rms_norm_amd


def torch_quantise_group(y):
    """torch's per-group quantisation of y on the CPU (binary32)."""
    yf = y.detach().cpu().float()
    rows, hidden = yf.shape
    g = yf.view(rows, hidden // 128, 128)
    sc = torch.clamp(g.abs().amax(-1, keepdim=True) / 448.0, min=torch.finfo(torch.float32).tiny)
    q = (g * (1.0 / sc)).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q.view(rows, hidden).view(torch.uint8).numpy(), sc.view(rows, -1).numpy()


def q_bits(q):
    return q.detach().cpu().contiguous().view(torch.uint8).numpy()


def same_floats(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return np.array_equal(a.view(np.uint32), b.view(np.uint32)) or np.array_equal(a, b, equal_nan=True)


def run_case(ops, rows, hidden, dtype, seed, dist="bench", eps=1e-6, special=False):
    from hp_rms_norm_amd import abi
    if special:
        x, r, w = special_inputs(rows, hidden, dtype, seed)
    else:
        x, r, w = make_inputs(rows, hidden, dtype, seed, dist)
    xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
    q, sc = ops.fused_add_rms_norm_fp8_group(xd, rd, wd, eps)
    # the same inputs through the 16-bit op with this form's lane mapping
    # (the same fp32 reduction order, hence the same y)
    cfg = lane_mapping(abi, abi.select_config(rows, hidden, DT[dtype], abi.MODE_FP8_GROUP))
    assert cfg.tier in (1, 2), cfg.as_tuple()
    y, r16 = x.to(DEV), r.to(DEV)
    abi.BENCH.fused_add_rmsnorm(y.data_ptr(), wd.data_ptr(), r16.data_ptr(), rows, hidden, hidden, hidden, DT[dtype],
                                eps, torch.cuda.current_stream().cuda_stream, cfg)
    torch.cuda.synchronize()
    tag = f"{rows}x{hidden} {dtype} seed {seed}"
    assert torch.equal(xd.cpu().view(torch.int16), x.view(torch.int16)), "input modified " + tag
    assert torch.equal(rd.view(torch.int16), r16.view(torch.int16)), "residual differs from the 16-bit op " + tag
    tq, tsc = torch_quantise_group(y)
    assert same_floats(sc.cpu().numpy(), tsc), "scales " + tag
    d = oracle.e4m3_ulp_distance(q_bits(q), tq)
    assert d.max() == 0, f"q differs from torch's quantisation of y: {tag}"
    oy, ores = oracle.fused_add_rmsnorm(bits(x), bits(w), bits(r), eps, DT[dtype],
                                        threads=min(16, oracle.max_threads()))
    assert_residual_exact(bits(rd), ores, dtype, "residual " + tag)
    scales = sc.cpu().numpy()
    assert_group_scales(scales, oy, 128, dtype, "scales " + tag)
    with np.errstate(divide="ignore"):
        assert_fp8_from_y_within_one_ulp(q_bits(q), oy, np.repeat(np.float32(1.0) / scales, 128, axis=1), dtype,
                                         "q " + tag)


def test_fp8_group_golden_through_torch_op(ops, golden):
    """torch's per-group quantisation of torch's own 16-bit output (golden
    vectors): the residual bit-exact, the scales those of a group maximum
    within one ulp of torch's, q the quantisation of a y within one 16-bit ulp
    of torch's output."""
    n = 0
    for name, c in golden.items():
        if c["kind"] != "fp8_group":
            continue
        dtype = torch.bfloat16 if c["dtype"] == "bf16" else torch.float16
        x, r, w = (from_bits(c[k], dtype).to(DEV) for k in ("x", "r", "w"))
        q, sc = ops.fused_add_rms_norm_fp8_group(x, r, w, c["eps"])
        torch.cuda.synchronize()
        assert_residual_exact(bits(r), c["res"], dtype, name)
        scales = sc.cpu().numpy()
        assert_group_scales(scales, c["out"], 128, dtype, name)
        with np.errstate(divide="ignore"):
            isc = np.repeat(np.float32(1.0) / scales, 128, axis=1)
        assert_fp8_from_y_within_one_ulp(q_bits(q), c["out"], isc, dtype, name)
        n += 1
    assert n >= 3


@pytest.mark.parametrize("rows,hidden,dtype", [
    (4096, 4096, torch.bfloat16), (4096, 8192, torch.bfloat16), (4096, 16384, torch.bfloat16),
    (4096, 32768, torch.bfloat16), (4096, 5120, torch.float16), (4096, 7168, torch.float16),
    (1, 4096, torch.bfloat16), (32, 8192, torch.bfloat16), (512, 4096, torch.bfloat16)],
    ids=lambda v: str(v).replace("torch.", ""))
def test_fp8_group_baseline_shapes(ops, rows, hidden, dtype):
    print("fp8 group case", rows, hidden, dtype, flush=True)
    run_case(ops, rows, hidden, dtype, seed=rows + hidden, dist="outliers" if rows <= 512 else "bench")


def test_fp8_group_every_table_entry(ops):
    """H at every breakpoint of the table this form takes (and one group
    below), with 1100 rows (the bandwidth rows) and 7 rows (the latency
    rows), both dtypes at a few."""
    for hidden in (128, 256, 512, 640, 1024, 1152, 2048, 3072, 3200, 4096, 5120, 6144, 8192, 12288, 16384, 16256,
                   24576, 32768, 65536):
        for rows in (1100, 7):
            print("fp8 group table", rows, hidden, flush=True)
            run_case(ops, rows, hidden, torch.bfloat16, seed=hidden + rows)
    for hidden in (1024, 4096, 16384):
        run_case(ops, 300, hidden, torch.float16, seed=hidden + 1)


def test_fp8_group_special_rows(ops):
    """Rows of special values (NaN, infinities, zero rows with eps = 0,
    binary32 overflow of the sum of squares, subnormals): a group holding NaN
    gets a NaN scale and NaN codes, a zero group the scale FLT_MIN and zero
    codes, as torch's quantisation of y."""
    for rows, hidden in ((28, 1024), (300, 4096), (40, 32768)):
        for eps in (0.0, 1e-6):
            print("fp8 group special", rows, hidden, eps, flush=True)
            run_case(ops, rows, hidden, torch.bfloat16, seed=rows + hidden, eps=eps, special=True)


def test_fp8_group_strided_misaligned_output_and_scales(ops):
    from hp_rms_norm_amd import abi
    rows, hidden, eps, dtype = 40, 2048, 1e-6, torch.bfloat16
    x, r, w = make_inputs(rows, hidden, dtype, 79)
    oy, ores = oracle.fused_add_rmsnorm(bits(x), bits(w), bits(r), eps, oracle.BF16)
    for offset, pad, spad in ((0, 64, 0), (1, 3, 5)):
        xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
        buf = torch.zeros(rows, hidden + pad + offset, dtype=torch.uint8, device=DEV)
        qv = buf[:, offset:offset + hidden]
        sbuf = torch.full((rows, hidden // 128 + spad), -1.0, dtype=torch.float32, device=DEV)
        sv = sbuf[:, :hidden // 128]
        abi.fused_add_rmsnorm_fp8_group(qv.data_ptr(), sv.data_ptr(), xd.data_ptr(), wd.data_ptr(), rd.data_ptr(),
                                        rows, hidden, qv.stride(0), sv.stride(0), 1, hidden, hidden, abi.DTYPE_BF16,
                                        eps, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert_residual_exact(bits(rd), ores, dtype)
        scales = sv.cpu().numpy()
        assert_group_scales(scales, oy, 128, dtype)
        assert_fp8_from_y_within_one_ulp(qv.cpu().numpy(), oy, np.repeat(np.float32(1.0) / scales, 128, axis=1),
                                         dtype)
        assert not buf[:, :offset].any() and not buf[:, offset + hidden:].any()
        assert (sbuf[:, hidden // 128:] == -1.0).all()


def test_fp8_group_of_one_group_rows_equals_the_per_row_form(ops):
    """With H = 128 a row is one group: q and the scales equal the per-row FP8
    form's (which takes another lane mapping, hence the comparison through y:
    both quantise their own y, and the two y agree within 1 ulp)."""
    rows, hidden = 512, 128
    x, r, w = make_inputs(rows, hidden, torch.bfloat16, 81)
    xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
    q, sc = ops.fused_add_rms_norm_fp8_group(xd, rd, wd, 1e-6)
    xd2, rd2 = x.to(DEV), r.to(DEV)
    q1, sc1 = ops.fused_add_rms_norm_fp8(xd2, rd2, wd, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(rd.view(torch.int16), rd2.view(torch.int16))
    assert oracle.e4m3_ulp_distance(q_bits(q), q_bits(q1)).max() <= 1
    np.testing.assert_allclose(sc.cpu().numpy().reshape(-1), sc1.cpu().numpy().reshape(-1), rtol=2.0 ** -7)


@pytest.mark.parametrize("rows,hidden,pad", [(4096, 4096, 0), (4093, 7168, 3), (1, 4096, 3), (37, 128, 0),
                                             (300, 16384, 1), (2049, 32768, 3)])
def test_fp8_group_column_major_scales_through_the_abi(ops, rows, hidden, pad):
    """Scales in the column-major (token-minor) layout: scale (r, g) at element
    g * (rows + pad) + r of a [groups, rows + pad] buffer; the same q, scales
    and residual as the row-major call, bit for bit (the layout does not change
    the kernel's shape), and the padding columns untouched."""
    from hp_rms_norm_amd import abi
    print("fp8 group column-major", rows, hidden, pad, flush=True)
    x, r, w = make_inputs(rows, hidden, torch.bfloat16, rows + hidden)
    st = torch.cuda.current_stream().cuda_stream
    ng = hidden // 128
    xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
    q = torch.empty(rows, hidden, dtype=torch.uint8, device=DEV)
    sb = torch.full((ng, rows + pad), -1.0, dtype=torch.float32, device=DEV)
    abi.fused_add_rmsnorm_fp8_group(q.data_ptr(), sb.data_ptr(), xd.data_ptr(), wd.data_ptr(), rd.data_ptr(), rows,
                                    hidden, hidden, 1, rows + pad, hidden, hidden, abi.DTYPE_BF16, 1e-6, st)
    xd2, rd2 = x.to(DEV), r.to(DEV)
    q2 = torch.empty(rows, hidden, dtype=torch.uint8, device=DEV)
    s2 = torch.empty(rows, ng, dtype=torch.float32, device=DEV)
    abi.fused_add_rmsnorm_fp8_group(q2.data_ptr(), s2.data_ptr(), xd2.data_ptr(), wd.data_ptr(), rd2.data_ptr(), rows,
                                    hidden, hidden, ng, 1, hidden, hidden, abi.DTYPE_BF16, 1e-6, st)
    torch.cuda.synchronize()
    assert torch.equal(q, q2) and torch.equal(rd.view(torch.int16), rd2.view(torch.int16))
    assert same_floats(sb[:, :rows].t().cpu().numpy(), s2.cpu().numpy())
    assert (sb[:, rows:] == -1.0).all()
    oy, ores = oracle.fused_add_rmsnorm(bits(x), bits(w), bits(r), 1e-6, oracle.BF16,
                                        threads=min(16, oracle.max_threads()))
    assert_residual_exact(bits(rd), ores, torch.bfloat16)
    scales = sb[:, :rows].t().cpu().numpy()
    assert_group_scales(scales, oy, 128, torch.bfloat16)
    assert_fp8_from_y_within_one_ulp(q_bits(q), oy, np.repeat(np.float32(1.0) / scales, 128, axis=1), torch.bfloat16)


def test_fp8_group_column_major_scales_through_the_torch_op(ops):
    """The allocating form with column-major scales, 16-byte aligned columns
    (tokens rounded up to a multiple of 4), on a [batch, seq, H] input; and the
    in-place form given a transposed view: both equal the row-major form."""
    b, s_, hidden = 3, 343, 5120
    x, r, w = make_inputs(b * s_, hidden, torch.bfloat16, 91)
    x, r = x.view(b, s_, hidden), r.view(b, s_, hidden)
    wd = w.to(DEV)
    xd, rd = x.to(DEV), r.to(DEV)
    q, sc = ops.fused_add_rms_norm_fp8_group(xd, rd, wd, 1e-6, column_major_scales=True, scale_row_align=4)
    assert sc.shape == (b, s_, hidden // 128) and sc.stride(-1) == -(-b * s_ // 4) * 4 and sc.stride(1) == 1
    xd2, rd2 = x.to(DEV), r.to(DEV)
    q2, sc2 = ops.fused_add_rms_norm_fp8_group(xd2, rd2, wd, 1e-6)
    xd3, rd3 = x.to(DEV), r.to(DEV)
    q3 = torch.empty_like(q)
    sc3 = torch.full((hidden // 128, b * s_), -1.0, device=DEV)
    ops.hp_rms_norm_fp8_group(q3, sc3.t().view(b, s_, hidden // 128), xd3, wd, rd3, 1e-6)
    torch.cuda.synchronize()
    for qq, ss, rr in ((q, sc, rd), (q3, sc3.t().view(b, s_, -1), rd3)):
        assert torch.equal(qq.view(torch.uint8), q2.view(torch.uint8))
        assert same_floats(ss.cpu().numpy(), sc2.cpu().numpy())
        assert torch.equal(rr.view(torch.int16), rd2.view(torch.int16))
