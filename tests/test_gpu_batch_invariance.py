"""Batch-invariant mode (hprms_set_batch_invariant): a row's output bits do
not depend on how many rows the call holds, as with the reference, whose
launcher chooses its kernel by the hidden size alone
(hp_rms_norm/csrc/cuda/hp_rms_norm.cuh:562-618).

Each test runs the same rows through row counts that, with the mode off,
select the latency, wide, one- and two-wave and bandwidth shapes (and the
small calls that drop sc1), and requires bit-identical residuals and
outputs with the mode on.  Parity with the oracle is tested elsewhere; this
is a property of the kernels against themselves.  The mode is restored after
each test.
"""
import numpy as np
import pytest
import torch

from helpers import DT, bits, make_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

# widths on the 128-byte grid, one or more per table row, and a few off it
WIDTHS = [128, 512, 1024, 1536, 2048, 2560, 3072, 3584, 4096, 5120, 6144, 7168, 8192, 9216, 9280, 12288, 14336,
          16384, 20480, 24576, 32768, 40960, 65536, 1000, 4100, 12289]
ROW_COUNTS = [1, 8, 64, 300, 700, 1024, 1500, 2048, 3000]


@pytest.fixture(scope="module")
def abi():
    assert torch.cuda.is_available(), "the gpu tests need a HIP device"
    import hp_rms_norm_amd  # noqa: F401  (registers the torch ops; fails loudly if unbuilt)
    from hp_rms_norm_amd import abi as a
    a.lib()
    return a


@pytest.fixture
def invariant(abi):
    import hp_rms_norm_amd
    previous = hp_rms_norm_amd.set_batch_invariant(True)
    assert hp_rms_norm_amd.batch_invariant() and abi.batch_invariant()
    yield
    hp_rms_norm_amd.set_batch_invariant(previous)


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _total(hidden):
    return min(4096, (1 << 26) // hidden)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_in_place_rows_do_not_depend_on_the_row_count(abi, invariant, dtype):
    import hp_rms_norm_amd
    for hidden in WIDTHS:
        total = _total(hidden)
        x, r, w = make_inputs(total, hidden, dtype, seed=hidden)
        wd = w.to(DEV)
        xf, rf = x.to(DEV), r.to(DEV)
        hp_rms_norm_amd.hp_rms_norm(xf, wd, rf, 1e-6)
        torch.cuda.synchronize()
        full_out, full_res = bits(xf), bits(rf)
        for rows in [n for n in ROW_COUNTS if n < total]:
            print(f"rows {rows} of {total} x {hidden} {dtype}", flush=True)
            xs, rs = x[:rows].to(DEV), r[:rows].to(DEV)
            hp_rms_norm_amd.hp_rms_norm(xs, wd, rs, 1e-6)
            torch.cuda.synchronize()
            assert np.array_equal(bits(rs), full_res[:rows]), f"residual, {rows} rows x {hidden}"
            diff = np.nonzero(bits(xs) != full_out[:rows])
            assert diff[0].size == 0, (f"{diff[0].size} outputs differ with {rows} rows x {hidden} (first at row "
                                       f"{diff[0][0]}, element {diff[1][0]})")


@pytest.mark.parametrize("form", ["plain", "out_of_place", "reduce", "fp8", "fp8_static", "fp8_group", "mxfp4"])
def test_other_forms_do_not_depend_on_the_row_count(abi, invariant, form):
    dtype = torch.bfloat16
    code = DT[dtype]
    for hidden in (1024, 2048, 4096, 6144, 8192, 9216, 16384, 32768):
        total = _total(hidden)
        x, r, w = make_inputs(total, hidden, dtype, seed=hidden + 2)
        xd, wd = x.to(DEV), w.to(DEV)

        def run(n):
            st = _stream()
            rd = r[:n].to(DEV)
            if form == "plain":
                od = torch.empty((n, hidden), dtype=dtype, device=DEV)
                abi.rmsnorm(od.data_ptr(), xd.data_ptr(), wd.data_ptr(), n, hidden, hidden, hidden, code, 1e-6, st)
                outs = [od]
            elif form == "out_of_place":
                od, rod = torch.empty((n, hidden), dtype=dtype, device=DEV), torch.empty((n, hidden), dtype=dtype,
                                                                                           device=DEV)
                abi.fused_add_rmsnorm_out(od.data_ptr(), rod.data_ptr(), xd.data_ptr(), rd.data_ptr(), wd.data_ptr(),
                                          n, hidden, hidden, hidden, hidden, hidden, code, 1e-6, st)
                outs = [od, rod]
            elif form == "reduce":
                od = torch.empty((n, hidden), dtype=dtype, device=DEV)
                abi.reduce_add_rmsnorm(od.data_ptr(), [xd.data_ptr(), xd.data_ptr()], wd.data_ptr(), rd.data_ptr(),
                                       n, hidden, hidden, hidden, hidden, code, 1e-6, st)
                outs = [od, rd]
            elif form == "fp8":
                q = torch.empty((n, hidden), dtype=torch.uint8, device=DEV)
                sc = torch.empty(n, dtype=torch.float32, device=DEV)
                abi.fused_add_rmsnorm_fp8(q.data_ptr(), sc.data_ptr(), xd.data_ptr(), wd.data_ptr(), rd.data_ptr(), n,
                                          hidden, hidden, hidden, hidden, code, 1e-6, st)
                outs = [q, sc, rd]
            elif form == "fp8_static":
                q = torch.empty((n, hidden), dtype=torch.uint8, device=DEV)
                sc = torch.full((1,), 0.02, dtype=torch.float32, device=DEV)
                abi.fused_add_rmsnorm_fp8_static(q.data_ptr(), sc.data_ptr(), xd.data_ptr(), wd.data_ptr(),
                                                 rd.data_ptr(), n, hidden, hidden, hidden, hidden, code, 1e-6, st)
                outs = [q, rd]
            elif form == "fp8_group":
                q = torch.empty((n, hidden), dtype=torch.uint8, device=DEV)
                sc = torch.empty((n, hidden // 128), dtype=torch.float32, device=DEV)
                abi.fused_add_rmsnorm_fp8_group(q.data_ptr(), sc.data_ptr(), xd.data_ptr(), wd.data_ptr(),
                                                rd.data_ptr(), n, hidden, hidden, hidden // 128, 1, hidden, hidden,
                                                code, 1e-6, st)
                outs = [q, sc, rd]
            else:
                q = torch.empty((n, hidden // 2), dtype=torch.uint8, device=DEV)
                s = torch.empty((n, hidden // 32), dtype=torch.uint8, device=DEV)
                abi.fused_add_rmsnorm_mx(q.data_ptr(), s.data_ptr(), xd.data_ptr(), wd.data_ptr(), rd.data_ptr(), n,
                                         hidden, hidden // 2, hidden // 32, hidden, hidden, abi.MX_FP4_E2M1, code,
                                         1e-6, st)
                outs = [q, s, rd]
            torch.cuda.synchronize()
            return [o.view(torch.uint8).cpu().numpy() for o in outs]

        full = run(total)
        for rows in [n for n in ROW_COUNTS if n < total]:
            print(f"{form} rows {rows} x {hidden}", flush=True)
            for k, (a, b) in enumerate(zip(run(rows), full)):
                assert np.array_equal(a, b[: a.shape[0]]), f"{form}: output {k}, {rows} rows x {hidden}"

