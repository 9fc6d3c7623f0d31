"""GPU parity of the fused add+RMSNorm with an FP8 (OCP e4m3fn) output and
per-row scales whose row maximum is bounded above (the activation scale bound
of FP8 row-wise checkpoints).

Pins: the residual is bit-exact against the oracle; q and the scales equal,
bit for bit, torch's bounded quantisation of the 16-bit output the same kernel
family produces for the same inputs (the 16-bit op run with the FP8 table's
lane mapping); every row the bound reaches gets exactly max(bound / 448,
FLT_MIN); the rows it does not reach equal the unbounded form's bytes.
`input` and the bound are not modified.  NaN encodings differ (hardware 0xFF,
torch 0x7F): NaN compares equal to NaN.
"""
import numpy as np
import pytest
import torch

from helpers import DT, assert_residual_exact, bits, lane_mapping, make_inputs, special_inputs
from oracle import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def ops():
    assert torch.cuda.is_available(), "the gpu tests need a HIP device"
    import hp_rms_norm_amd
    return hp_rms_norm_amd


def torch_quantise_ub(y, scale_ub):
    """torch's bounded per-row quantisation of y on the CPU (binary32)."""
    yf = y.detach().cpu().float()
    amax = yf.abs().amax(-1, keepdim=True)
    ub = torch.tensor(scale_ub, dtype=torch.float32)
    amax = torch.where(amax > ub, ub, amax)
    sc = torch.clamp(amax / 448.0, min=torch.finfo(torch.float32).tiny)
    q = (yf * (1.0 / sc)).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q.view(torch.uint8).numpy(), sc.view(-1).numpy()


def q_bits(q):
    return q.detach().cpu().contiguous().view(torch.uint8).numpy()


def same_floats(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return np.array_equal(a.view(np.uint32), b.view(np.uint32)) or np.array_equal(a, b, equal_nan=True)


def run_case(ops, rows, hidden, dtype, seed, ub, special=False):
    from hp_rms_norm_amd import abi
    x, r, w = special_inputs(rows, hidden, dtype, seed) if special else make_inputs(rows, hidden, dtype, seed)
    xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
    ubd = torch.tensor([ub], dtype=torch.float32, device=DEV)
    q, sc = ops.fused_add_rms_norm_fp8(xd, rd, wd, 1e-6, scale_ub=ubd)
    # the unbounded form and the 16-bit op with the same lane mapping, on fresh copies
    xd2, rd2 = x.to(DEV), r.to(DEV)
    q0, sc0 = ops.fused_add_rms_norm_fp8(xd2, rd2, wd, 1e-6)
    cfg = lane_mapping(abi, abi.select_config(rows, hidden, DT[dtype], abi.MODE_FP8))
    y, r16 = x.to(DEV), r.to(DEV)
    abi.BENCH.fused_add_rmsnorm(y.data_ptr(), wd.data_ptr(), r16.data_ptr(), rows, hidden, hidden, hidden, DT[dtype],
                                1e-6, torch.cuda.current_stream().cuda_stream, None if cfg.tier == 3 else cfg)
    torch.cuda.synchronize()
    tag = f"{rows}x{hidden} {dtype} seed {seed} bound {ub}"
    assert torch.equal(xd.cpu().view(torch.int16), x.view(torch.int16)), "input modified " + tag
    assert ubd.item() == float(np.float32(ub)) or (np.isnan(ub) and np.isnan(ubd.item())), "bound modified " + tag
    assert torch.equal(rd.view(torch.int16), r16.view(torch.int16)), "residual differs from the 16-bit op " + tag
    tq, tsc = torch_quantise_ub(y, ub)
    scn = sc.reshape(-1).cpu().numpy()
    assert same_floats(scn, tsc), "scales " + tag
    assert oracle.e4m3_ulp_distance(q_bits(q), tq).max() == 0, "q " + tag
    yf = y.cpu().float().abs().amax(-1).numpy()
    with np.errstate(invalid="ignore"):
        bounded = yf > np.float32(ub)
    want = max(np.float32(np.float32(ub) / np.float32(448.0)), np.float32(np.finfo(np.float32).tiny))
    assert (scn[bounded] == want).all(), "bounded scales " + tag
    free = ~bounded
    assert same_floats(scn[free], sc0.reshape(-1).cpu().numpy()[free]), "unbounded rows' scales " + tag
    assert np.array_equal(q_bits(q)[free], q_bits(q0)[free]) or \
        oracle.e4m3_ulp_distance(q_bits(q)[free], q_bits(q0)[free]).max() == 0, "unbounded rows' q " + tag
    _, ores = oracle.fused_add_rmsnorm(bits(x), bits(w), bits(r), 1e-6, DT[dtype],
                                       threads=min(16, oracle.max_threads()))
    assert_residual_exact(bits(rd), ores, dtype, "residual " + tag)
    return int(bounded.sum())


@pytest.mark.parametrize("rows,hidden,dtype", [
    (4096, 4096, torch.bfloat16), (4096, 8192, torch.bfloat16), (4096, 16384, torch.bfloat16),
    (4096, 32768, torch.bfloat16), (4096, 5120, torch.float16), (1, 4096, torch.bfloat16),
    (7, 8192, torch.bfloat16), (300, 1000, torch.bfloat16), (16, 70000, torch.bfloat16), (37, 13, torch.float16)],
    ids=lambda v: str(v).replace("torch.", ""))
def test_fp8_ub_shapes(ops, rows, hidden, dtype):
    """The table's rows, the latency rows, odd widths and the general kernels,
    with a bound that reaches most rows, some rows, and none."""
    print("fp8 ub case", rows, hidden, dtype, flush=True)
    reached = [run_case(ops, rows, hidden, dtype, rows + hidden, ub) for ub in (2.0, 3.6, float("inf"))]
    assert reached[2] == 0 and reached[0] >= reached[1] and (rows < 16 or reached[0] > 0), reached


def test_fp8_ub_special_rows_and_bounds(ops):
    """Rows of special values (a row holding NaN keeps a NaN scale), and bounds
    that are zero, subnormal, huge and NaN (which bounds nothing)."""
    for rows, hidden in ((28, 1024), (300, 4096), (16, 70000)):
        for ub in (0.0, 2.0 ** -140, 1.0, 1e30, float("nan")):
            print("fp8 ub special", rows, hidden, ub, flush=True)
            run_case(ops, rows, hidden, torch.bfloat16, rows + hidden, ub, special=True)


def test_fp8_ub_through_the_c_abi_and_its_checks(ops):
    from hp_rms_norm_amd import abi
    rows, hidden = 64, 4096
    x, r, w = (t.to(DEV) for t in make_inputs(rows, hidden, torch.bfloat16, 3))
    q = torch.empty(rows, hidden, dtype=torch.uint8, device=DEV)
    sc = torch.empty(rows, dtype=torch.float32, device=DEV)
    ub = torch.tensor([2.5], device=DEV)
    st = torch.cuda.current_stream().cuda_stream
    with pytest.raises(abi.HprmsError):
        abi.fused_add_rmsnorm_fp8_ub(q.data_ptr(), sc.data_ptr(), 0, x.data_ptr(), w.data_ptr(), r.data_ptr(), rows,
                                     hidden, hidden, hidden, hidden, abi.DTYPE_BF16, 1e-6, st)
    abi.fused_add_rmsnorm_fp8_ub(q.data_ptr(), sc.data_ptr(), ub.data_ptr(), x.data_ptr(), w.data_ptr(),
                                 r.data_ptr(), rows, hidden, hidden, hidden, hidden, abi.DTYPE_BF16, 1e-6, st)
    torch.cuda.synchronize()
    assert (sc <= np.float32(2.5) / np.float32(448.0)).all()
