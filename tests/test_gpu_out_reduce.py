"""GPU parity of the out-of-place fused op and of the partial-sum form
(reduce + residual-add + RMSNorm) against the CPU oracle, through the C ABI
and the torch ops.

Bar: the residual (and the residual output) bit-exact, the normalised output
within 1 ulp and atol = rtol = 1e-2 of the oracle.  Both forms share the
table with the in-place op, so with the same inputs their outputs must also be
bit-identical to the in-place op's (same reduction order).
"""
import numpy as np
import pytest
import torch

from helpers import DT, as_dispatched, assert_output_close, assert_residual_exact, bits, make_inputs, oracle_fused
from oracle import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

# every bandwidth row of the table (rows = 513) and every latency row (rows = 64),
# with a ragged width below each boundary
HIDDENS = [128, 256, 512, 1000, 2048, 3064, 4096, 8192, 12280, 16384, 24576, 32768, 65536]


@pytest.fixture(scope="module")
def abi():
    assert torch.cuda.is_available(), "the gpu tests need a HIP device"
    import hp_rms_norm_amd  # noqa: F401  (registers the torch ops; fails loudly if unbuilt)
    from hp_rms_norm_amd import abi as a
    a.lib()
    return a


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _stride(t):
    return t.stride(0) if t.shape[0] > 1 else t.shape[1]


def in_place(abi, x, r, w, eps, config):
    """The in-place op forced to `config` (through the C ABI of the bench
    library, which also holds the other forms' shapes as in-place kernels)."""
    xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
    abi.BENCH.fused_add_rmsnorm(xd.data_ptr(), wd.data_ptr(), rd.data_ptr(), xd.shape[0], xd.shape[1], _stride(xd),
                                _stride(rd), DT[xd.dtype], eps, _stream(), config)
    torch.cuda.synchronize()
    return bits(xd), bits(rd)


# ---- out of place ----------------------------------------------------------------------
def run_out(abi, xd, rd, wd, od, rod, eps):
    abi.fused_add_rmsnorm_out(od.data_ptr(), rod.data_ptr(), xd.data_ptr(), rd.data_ptr(), wd.data_ptr(),
                              xd.shape[0], xd.shape[1], _stride(od), _stride(rod), _stride(xd), _stride(rd),
                              DT[xd.dtype], eps, _stream())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_out_of_place_every_table_row(abi, dtype):
    for rows in (513, 64):
        for hidden in HIDDENS:
            print("out", rows, hidden, dtype, flush=True)
            x, r, w = make_inputs(rows, hidden, dtype, seed=rows + hidden)
            want_out, want_res = oracle_fused(x, r, w, 1e-6, dtype)
            xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
            od, rod = torch.empty_like(xd), torch.empty_like(rd)
            run_out(abi, xd, rd, wd, od, rod, 1e-6)
            torch.cuda.synchronize()
            tag = f"{rows}x{hidden} {dtype}"
            assert np.array_equal(bits(xd), bits(x)) and np.array_equal(bits(rd), bits(r)), "inputs modified " + tag
            assert_residual_exact(bits(rod), want_res, dtype, "residual_out " + tag)
            assert_output_close(bits(od), want_out, dtype, "out " + tag)
            # the in-place op run with the configuration the out-of-place form chose (the
            # two forms' tables differ at some row counts), in the variant the dispatch
            # runs on these rows, gives the same bits
            c_out = as_dispatched(abi, abi.select_config(rows, hidden, DT[dtype], abi.MODE_OUT), hidden)
            ip_out, ip_res = in_place(abi, x, r, w, 1e-6, c_out)
            assert np.array_equal(bits(od), ip_out), "differs from the in-place op " + tag
            assert np.array_equal(bits(rod), ip_res), "residual differs from the in-place op " + tag


# the wide rows of 1K-3K (32 lanes x ceil(H / 256) vectors, two rows per one-wave
# workgroup) at row counts the dispatch gives them, on and off the 128-byte grid
WIDE_CASES = [(1280, 1032), (1536, 2048), (4096, 1536), (2048, 2560), (3072, 2304), (1100, 1288), (4096, 2049),
              (4096, 3072), (1600, 2817), (2000, 3064)]


# one row per one-wave workgroup (64 lanes) at 3K-5K, 768 < rows <= 2048, and one row per
# two-wave workgroup (128 lanes) at 5K-8K, 512 < rows <= 1280
WAVE_CASES = [(1000, 4096, 64), (2048, 3584, 64), (800, 5120, 64), (1024, 6144, 128), (600, 8192, 128)]


@pytest.mark.parametrize("rows,hidden,lanes", [c + (32,) for c in WIDE_CASES] + WAVE_CASES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_wide_rows_in_and_out_of_place(abi, rows, hidden, lanes, dtype):
    print("wide", rows, hidden, dtype, flush=True)
    for mode in (abi.MODE_FUSED, abi.MODE_OUT):
        c = abi.select_config(rows, hidden, DT[dtype], mode)
        assert (c.lanes_per_row, c.block_threads) == (lanes, max(lanes, 64)), (mode, c.as_tuple())
    x, r, w = make_inputs(rows, hidden, dtype, seed=rows + hidden)
    want_out, want_res = oracle_fused(x, r, w, 1e-6, dtype)
    xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
    od, rod = torch.empty_like(xd), torch.empty_like(rd)
    run_out(abi, xd, rd, wd, od, rod, 1e-6)
    torch.cuda.synchronize()
    tag = f"{rows}x{hidden} {dtype}"
    assert np.array_equal(bits(xd), bits(x)) and np.array_equal(bits(rd), bits(r)), "inputs modified " + tag
    assert_residual_exact(bits(rod), want_res, dtype, "residual_out " + tag)
    assert_output_close(bits(od), want_out, dtype, "out " + tag)
    # the in-place op through its own dispatch: the same shape, so the same bits
    abi.fused_add_rmsnorm(xd.data_ptr(), wd.data_ptr(), rd.data_ptr(), rows, hidden, hidden, hidden, DT[dtype],
                          1e-6, _stream())
    torch.cuda.synchronize()
    assert_residual_exact(bits(rd), want_res, dtype, "residual " + tag)
    assert np.array_equal(bits(xd), bits(od)), "in place differs from out of place " + tag
    assert np.array_equal(bits(rd), bits(rod)), "residual differs from out of place " + tag


def test_out_of_place_torch_ops_and_aliases(abi):
    import hp_rms_norm_amd
    x, r, w = make_inputs(300, 4096, torch.bfloat16, seed=5)
    want_out, want_res = oracle_fused(x, r, w, 1e-6, torch.bfloat16)
    xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
    out, res = hp_rms_norm_amd.fused_add_rms_norm(xd, rd, wd, 1e-6)       # allocating form
    torch.cuda.synchronize()
    assert_residual_exact(bits(res), want_res, torch.bfloat16)
    assert_output_close(bits(out), want_out, torch.bfloat16)
    assert np.array_equal(bits(xd), bits(x)) and np.array_equal(bits(rd), bits(r))
    # the out form with out = input and residual_out = residual is the in-place op
    hp_rms_norm_amd.fused_add_rms_norm_out(xd, rd, xd, wd, rd, 1e-6)
    torch.cuda.synchronize()
    assert np.array_equal(bits(xd), bits(out)) and np.array_equal(bits(rd), bits(res))
    # input and residual may be the same tensor when both are only read: s = x + x
    y = x.to(DEV)
    o2, s2 = hp_rms_norm_amd.fused_add_rms_norm(y, y, wd, 1e-6)
    want_out2, want_res2 = oracle_fused(x, x, w, 1e-6, torch.bfloat16)
    torch.cuda.synchronize()
    assert_residual_exact(bits(s2), want_res2, torch.bfloat16)
    assert_output_close(bits(o2), want_out2, torch.bfloat16)


@pytest.mark.parametrize("hidden,pad", [(1001, 3), (4096, 24), (4096, 3), (6143, 1), (11001, 5), (16383, 1),
                                        (20001, 2)])
def test_out_of_place_strided_and_odd_widths(abi, hidden, pad):
    dtype = torch.float16
    rows = 37
    x, r, w = make_inputs(rows, hidden, dtype, seed=hidden + pad)
    want_out, want_res = oracle_fused(x, r, w, 1e-6, dtype)
    wide = lambda: torch.zeros(rows, hidden + pad, dtype=dtype, device=DEV)   # noqa: E731
    xb, rb, ob, rob = wide(), wide(), wide(), wide()
    xd, rd = xb[:, pad:pad + hidden], rb[:, :hidden]
    xd.copy_(x.to(DEV))
    rd.copy_(r.to(DEV))
    od, rod = ob[:, :hidden], rob[:, pad:pad + hidden]
    run_out(abi, xd, rd, w.to(DEV), od, rod, 1e-6)
    torch.cuda.synchronize()
    assert_residual_exact(bits(rod), want_res, dtype)
    assert_output_close(bits(od), want_out, dtype)
    assert not bits(ob[:, hidden:]).any() and not bits(rob[:, :pad]).any(), "wrote outside the rows"


# ---- partial sums ----------------------------------------------------------------------
def make_parts(nparts, rows, hidden, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn((rows, hidden), generator=g).to(dtype) for _ in range(nparts)]


def oracle_reduce(parts, r, w, eps, dtype):
    hidden = r.shape[-1]
    return oracle.reduce_add_rmsnorm([bits(p).reshape(-1, hidden) for p in parts], bits(w),
                                     bits(r).reshape(-1, hidden), eps, DT[dtype], threads=min(16, oracle.max_threads()))


def run_reduce(abi, od, pds, wd, rd, eps):
    abi.reduce_add_rmsnorm(od.data_ptr(), [p.data_ptr() for p in pds], wd.data_ptr(), rd.data_ptr(), rd.shape[0],
                           rd.shape[1], _stride(od), _stride(pds[0]), _stride(rd), DT[rd.dtype], eps, _stream())


@pytest.mark.parametrize("nparts", [1, 2, 3, 8])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_reduce_every_table_row(abi, dtype, nparts):
    for rows in (513, 64):
        for hidden in HIDDENS:
            if nparts == 8 and hidden > 16384 and rows == 513:
                continue   # keeps the oracle's share of the test short; covered by the nparts = 3 case
            print("reduce", nparts, rows, hidden, dtype, flush=True)
            parts = make_parts(nparts, rows, hidden, dtype, seed=nparts * 1000 + hidden)
            _, r, w = make_inputs(rows, hidden, dtype, seed=rows + hidden)
            want_out, want_res = oracle_reduce(parts, r, w, 1e-6, dtype)
            pds = [p.to(DEV) for p in parts]
            rd, wd = r.to(DEV), w.to(DEV)
            od = torch.empty_like(rd)
            run_reduce(abi, od, pds, wd, rd, 1e-6)
            torch.cuda.synchronize()
            tag = f"P={nparts} {rows}x{hidden} {dtype}"
            assert all(np.array_equal(bits(pd), bits(p)) for pd, p in zip(pds, parts)), "parts modified " + tag
            assert_residual_exact(bits(rd), want_res, dtype, "residual " + tag)
            assert_output_close(bits(od), want_out, dtype, "out " + tag)
            if nparts == 1:
                # the in-place op with the reduce form's shape and variant (the same fp32
                # summation order)
                cfg = as_dispatched(abi, abi.select_config(rows, hidden, DT[dtype], abi.MODE_REDUCE), hidden)
                cfg.flags &= ~32768   # (the partial sums' part prefetch: no in-place counterpart)
                xd, rd2 = parts[0].to(DEV), r.to(DEV)
                abi.BENCH.fused_add_rmsnorm(xd.data_ptr(), wd.data_ptr(), rd2.data_ptr(), rows, hidden, hidden, hidden,
                                            DT[dtype], 1e-6, _stream(), cfg)
                torch.cuda.synchronize()
                assert np.array_equal(bits(od), bits(xd)), "P=1 differs from the in-place op " + tag
                assert np.array_equal(bits(rd), bits(rd2)), "P=1 residual differs from the in-place op " + tag


def test_reduce_torch_op_out_is_a_part(abi):
    import hp_rms_norm_amd
    parts = make_parts(4, 200, 8192, torch.bfloat16, seed=11)
    _, r, w = make_inputs(200, 8192, torch.bfloat16, seed=12)
    want_out, want_res = oracle_reduce(parts, r, w, 1e-6, torch.bfloat16)
    pds = [p.to(DEV) for p in parts]
    rd = r.to(DEV)
    hp_rms_norm_amd.reduce_add_rms_norm(pds[0], pds, w.to(DEV), rd, 1e-6)
    torch.cuda.synchronize()
    assert_residual_exact(bits(rd), want_res, torch.bfloat16)
    assert_output_close(bits(pds[0]), want_out, torch.bfloat16)


@pytest.mark.parametrize("hidden,pad", [(1001, 3), (4096, 24), (7167, 1), (12289, 7), (16383, 1), (20001, 2)])
def test_reduce_strided_and_odd_widths(abi, hidden, pad):
    dtype = torch.bfloat16
    rows = 29
    parts = make_parts(3, rows, hidden, dtype, seed=hidden)
    _, r, w = make_inputs(rows, hidden, dtype, seed=hidden + 1)
    want_out, want_res = oracle_reduce(parts, r, w, 1e-6, dtype)
    pbufs = [torch.zeros(rows, hidden + pad, dtype=dtype, device=DEV) for _ in parts]
    pds = [b[:, pad:pad + hidden] for b in pbufs]
    for pd, p in zip(pds, parts):
        pd.copy_(p.to(DEV))
    rb = torch.zeros(rows, hidden + pad, dtype=dtype, device=DEV)
    rd = rb[:, :hidden]
    rd.copy_(r.to(DEV))
    ob = torch.zeros(rows, hidden + 2 * pad, dtype=dtype, device=DEV)
    od = ob[:, pad:pad + hidden]
    run_reduce(abi, od, pds, w.to(DEV), rd, 1e-6)
    torch.cuda.synchronize()
    assert_residual_exact(bits(rd), want_res, dtype)
    assert_output_close(bits(od), want_out, dtype)
    assert not bits(ob[:, :pad]).any() and not bits(ob[:, pad + hidden:]).any(), "wrote outside the rows"


def test_reduce_full_size_identities(abi):
    """At the benchmark's size, checks that need no oracle: parts [x, 0, 0, 0]
    and [x/2, x/2] (exact halves) both sum to x exactly, so both must equal the
    in-place op on x bit for bit; rows are independent, so a permutation of the
    rows permutes the output."""
    import hp_rms_norm_amd
    rows, hidden = 4096, 8192
    x, r, w = (t.to(DEV) for t in make_inputs(rows, hidden, torch.bfloat16, seed=21))
    want_x, want_r = x.clone(), r.clone()
    # the in-place op with the reduce form's shape (the same fp32 summation order)
    cfg = abi.select_config(rows, hidden, abi.DTYPE_BF16, abi.MODE_REDUCE)
    abi.BENCH.fused_add_rmsnorm(want_x.data_ptr(), w.data_ptr(), want_r.data_ptr(), rows, hidden, hidden, hidden,
                                abi.DTYPE_BF16, 1e-6, _stream(), cfg)
    zeros = torch.zeros_like(x)
    for parts in ([x, zeros, zeros, zeros], [x * 0.5, x * 0.5]):
        rd = r.clone()
        out = torch.empty_like(x)
        hp_rms_norm_amd.reduce_add_rms_norm(out, parts, w, rd, 1e-6)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want_x.view(torch.int16))
        assert torch.equal(rd.view(torch.int16), want_r.view(torch.int16))
    perm = torch.randperm(rows, generator=torch.Generator().manual_seed(3)).to(DEV)
    parts = [torch.randn(rows, hidden, device=DEV).to(torch.bfloat16) for _ in range(3)]
    rd, rp = r.clone(), r[perm].clone()
    out, outp = torch.empty_like(x), torch.empty_like(x)
    hp_rms_norm_amd.reduce_add_rms_norm(out, parts, w, rd, 1e-6)
    hp_rms_norm_amd.reduce_add_rms_norm(outp, [p[perm].contiguous() for p in parts], w, rp, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(outp.view(torch.int16), out[perm].view(torch.int16))
    assert torch.equal(rp.view(torch.int16), rd[perm].view(torch.int16))


def test_graph_capture_and_replay_of_both_forms(abi):
    """Both ops allocate nothing and issue no memset, so they can be captured
    together; every replay (fresh inputs copied in, eager work and syncs in
    between) must equal the eager result bit for bit."""
    import hp_rms_norm_amd
    rows, hidden, eps, dtype = 192, 8192, 1e-6, torch.bfloat16
    w = make_inputs(1, hidden, dtype, 0)[2].to(DEV)
    x, r = torch.empty(rows, hidden, dtype=dtype, device=DEV), torch.empty(rows, hidden, dtype=dtype, device=DEV)
    out, res_out = torch.empty_like(x), torch.empty_like(x)
    parts = [torch.empty_like(x) for _ in range(3)]
    r2, out2 = torch.empty_like(x), torch.empty_like(x)
    for t in (x, r, r2, *parts):
        t.normal_()

    def body():
        hp_rms_norm_amd.fused_add_rms_norm_out(out, res_out, x, w, r, eps)
        hp_rms_norm_amd.reduce_add_rms_norm(out2, parts, w, r2, eps)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        body()  # warm-up outside the graph
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        body()
    for rep in range(4):
        g = torch.Generator(device=DEV).manual_seed(50 + rep)
        fresh = {name: torch.randn(rows, hidden, device=DEV, generator=g).to(dtype)
                 for name in ("x", "r", "r2", "p0", "p1", "p2")}
        for dst, name in ((x, "x"), (r, "r"), (r2, "r2"), (parts[0], "p0"), (parts[1], "p1"), (parts[2], "p2")):
            dst.copy_(fresh[name])
        graph.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in (out, res_out, out2, r2)]
        e_out, e_res = hp_rms_norm_amd.fused_add_rms_norm(fresh["x"], fresh["r"], w, eps)
        e_r2, e_out2 = fresh["r2"].clone(), torch.empty_like(x)
        hp_rms_norm_amd.reduce_add_rms_norm(e_out2, [fresh["p0"], fresh["p1"], fresh["p2"]], w, e_r2, eps)
        torch.cuda.synchronize()
        for a, b, what in zip(got, (e_out, e_res, e_out2, e_r2), ("out", "residual_out", "reduce out", "reduce residual")):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"replay {rep}: {what}"
