"""GPU parity of the fused residual-add + RMSNorm kernels against the CPU oracle.

Bar (from the target): the residual is bit-exact, the normalised output is
within 1 ulp (and atol = rtol = 1e-2) of the oracle, fp32 accumulation.
Most tests call the kernels through the C ABI (hp_rms_norm_amd.abi, ctypes);
the drop-in torch op is covered by the golden, sweep and graph tests.
"""
import random

import numpy as np
import pytest
import torch

from helpers import (DT, assert_output_close, assert_residual_exact, bits, from_bits, make_inputs,
                     oracle_fused)
from oracle import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def abi():
    assert torch.cuda.is_available(), "the gpu tests need a HIP device"
    import hp_rms_norm_amd  # noqa: F401  (registers the torch ops; fails loudly if unbuilt)
    from hp_rms_norm_amd import abi as a
    a.lib()
    return a


def _stream():
    return torch.cuda.current_stream().cuda_stream


def run_abi(abi, x, w, r, eps, config=None):
    """x, r: device tensors viewed as [rows, hidden] with unit inner stride."""
    hidden = x.shape[-1]
    x2, r2 = x.view(-1, hidden), r.view(-1, hidden)
    abi.fused_add_rmsnorm(x2.data_ptr(), w.data_ptr(), r2.data_ptr(), x2.shape[0], hidden,
                          x2.stride(0) if x2.shape[0] > 1 else hidden,
                          r2.stride(0) if r2.shape[0] > 1 else hidden,
                          DT[x.dtype], eps, _stream(), config)


def check_case(abi, rows, hidden, dtype, eps=1e-6, seed=0, dist="bench", config=None, via="abi"):
    x, r, w = make_inputs(rows, hidden, dtype, seed, dist)
    want_out, want_res = oracle_fused(x, r, w, eps, dtype)
    xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
    if via == "abi":
        run_abi(abi, xd, wd, rd, eps, config)
    else:
        import hp_rms_norm_amd
        hp_rms_norm_amd.hp_rms_norm(xd, wd, rd, eps)
    torch.cuda.synchronize()
    tag = f"{rows}x{hidden} {dtype} seed {seed} {dist} cfg {config.as_tuple() if config else 'table'}"
    assert_residual_exact(bits(rd), want_res, dtype, "residual " + tag)
    return assert_output_close(bits(xd), want_out, dtype, "output " + tag)


# ---- golden vectors (the reference's own formula, evaluated by torch on CPU) ----
def test_golden_fused_through_torch_op(abi, golden):
    import hp_rms_norm_amd
    for name, c in golden.items():
        if c["kind"] != "fused":
            continue
        dtype = torch.bfloat16 if c["dtype"] == "bf16" else torch.float16
        x, r, w = (from_bits(c[k], dtype).to(DEV) for k in ("x", "r", "w"))
        print("golden", name, flush=True)
        hp_rms_norm_amd.hp_rms_norm(x, w, r, c["eps"])
        torch.cuda.synchronize()
        assert_residual_exact(bits(r), c["res"], dtype, name + " residual")
        assert_output_close(bits(x), c["out"], dtype, name + " output")


# ---- BASELINE.json's configurations --------------------------------------------------
C1 = [(4096, 4096, torch.bfloat16, "bench")]
C2 = [(4096, h, torch.bfloat16, "bench") for h in range(1024, 12288 + 1, 1024)]
C3 = [(4096, h, torch.bfloat16, "bench") for h in (13312, 14336, 16384, 20480, 24576, 28672, 32768)]
C4 = [(b, h, torch.bfloat16, "outliers") for b in (1, 8, 32, 128, 512) for h in (4096, 8192)]
C5 = [(4096, 5120, torch.float16, "bench"), (4096, 7168, torch.float16, "bench")]


@pytest.mark.parametrize("rows,hidden,dtype,dist", C1 + C2 + C3 + C4 + C5,
                         ids=lambda v: str(v).replace("torch.", ""))
def test_baseline_configs(abi, rows, hidden, dtype, dist):
    print("case", rows, hidden, dtype, dist, flush=True)
    d = check_case(abi, rows, hidden, dtype, seed=rows * 7 + hidden, dist=dist)
    # the only differences left are fp32 reduction order: rare 1-ulp flips
    assert (d != 0).mean() < 1e-3


def test_reference_sweep_through_torch_op(abi):
    """The reference test's sweep (test/test_hp_rms_norm.py:49-60): H = 128 ...
    32768 step 128, random token counts, eps = bf16 eps, N(0, 0.1) inputs; here
    seeded, smaller token counts, and both dtypes (the reference's loop only
    ever ran bf16)."""
    rng = random.Random(1234)
    eps = torch.finfo(torch.bfloat16).eps
    for dtype in (torch.bfloat16, torch.float16):
        for hidden in range(128, 32768 + 128, 128):
            rows = rng.randint(1, 48)
            check_case(abi, rows, hidden, dtype, eps=eps, seed=hidden, dist="reference_test", via="torch")


# ---- every built kernel configuration, with ragged row groups and tails -------------
def _configs(abi, dtype, mode=0):
    return abi.kernel_configs(DT[dtype], mode)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_every_kernel_config(abi, dtype):
    for cfg in _configs(abi, dtype):
        cover = cfg.lanes_per_row * cfg.vec_per_lane * 8
        rpb = cfg.block_threads // cfg.lanes_per_row
        hiddens = {cover, max(8, cover - 8), max(8, cover - cfg.lanes_per_row * 8 + 8)}
        for hidden in sorted(hiddens):
            rows = 3 * rpb + 1
            print("config", cfg.as_tuple(), "hidden", hidden, "rows", rows, flush=True)
            check_case(abi, rows, hidden, dtype, seed=hidden + rows, config=cfg)


def test_persistent_grid(abi):
    from hp_rms_norm_amd.abi import Config
    base = abi.select_config(1000, 4096, DT[torch.bfloat16])
    for grid in (1, 7, 64):
        cfg = Config(*base.as_tuple())
        cfg.grid_blocks = grid
        check_case(abi, 1000, 4096, torch.bfloat16, seed=grid, config=cfg)


@pytest.mark.parametrize("hidden", [12289, 16391])
def test_persistent_grid_weight_staged_in_lds(abi, hidden):
    """A persistent grid over a tail variant that stages the weight in LDS
    (flags bit 14; rows of odd width, each shifted by its own amount): every
    workgroup stages the weight in its first row group and reads it there for
    all its later ones."""
    from hp_rms_norm_amd.abi import Config
    base = abi.select_config(1024, hidden, DT[torch.bfloat16])
    assert base.flags & 16384, base.as_tuple()
    for grid in (1, 7, 64):
        cfg = Config(*base.as_tuple())
        cfg.grid_blocks = grid
        check_case(abi, 1024, hidden, torch.bfloat16, seed=grid + hidden, config=cfg)


# one row per one-wave workgroup: the in-place op at 3K-5K, on the 128-byte grid, from the
# latency rows' limit up to 2048 rows
# (64 lanes), and one row per two-wave workgroup at 5K-8K, 512 < rows <= 1280 (128 lanes)
@pytest.mark.parametrize("rows,hidden,lanes", [(1000, 4096, 64), (1536, 3584, 64), (2048, 5120, 64),
                                               (800, 4608, 64), (1024, 6144, 128), (600, 8192, 128),
                                               (1280, 5248, 128)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_wave_rows_through_the_table(abi, rows, hidden, lanes, dtype):
    c = abi.select_config(rows, hidden, DT[dtype])
    assert (c.lanes_per_row, c.block_threads) == (lanes, lanes), c.as_tuple()
    check_case(abi, rows, hidden, dtype, seed=rows + hidden)


# ---- odd widths, misalignment, row strides, the general tier --------------------------
# odd widths (the vector tiers' tail variants from 8 up, the general tier below 8 and above
# 65543) on both sides of the table's rows and of the general kernels' block sizes
@pytest.mark.parametrize("hidden", [1, 7, 13, 100, 255, 257, 1023, 1025, 4095, 4097, 16383, 16385, 40000])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_hidden_not_multiple_of_8(abi, hidden, dtype):
    check_case(abi, 37, hidden, dtype, seed=hidden)


# The register-resident general kernel's dispatch (hprms_general.hip): block size and
# the element-slot counts E it is instantiated for, per width range.
GENERAL_TIERS = ((64, 0, 1024, (1, 2, 3, 4, 5, 6, 7, 8, 10, 12, 14, 16)),
                 (256, 1024, 8192, (5, 6, 7, 8, 10, 12, 14, 16, 20, 24, 28, 32)),
                 (1024, 8192, 16384, (10, 12, 14, 16)))


def general_widths():
    """Odd widths at both ends of every (block, E) shape: the smallest width
    that needs E slots per thread and the largest that E slots hold."""
    out = []
    for block, lo, hi, slots in GENERAL_TIERS:
        prev = lo
        for e in slots:
            top = min(e * block, hi)
            out += [(prev + 1, block, e), (top - 1, block, e)]
            prev = top
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_general_every_slot_count(abi, dtype):
    """The general tier forced (the table sends these widths to the vector
    tiers' tail variants)."""
    from hp_rms_norm_amd.abi import Config
    general = Config(3, 256, 0, 0, 256, 0, 0)
    for hidden, block, e in general_widths():
        print("general slots", hidden, block, e, dtype, flush=True)
        check_case(abi, 23, hidden, dtype, seed=hidden + 1, config=general)


@pytest.mark.parametrize("rows,hidden", [(9, 100000), (2, 1 << 24)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_hidden_beyond_the_vector_tiers(abi, rows, hidden, dtype):
    """H > 65536 takes the general kernel, up to the documented maximum 2^24."""
    print("large hidden", rows, hidden, dtype, flush=True)
    check_case(abi, rows, hidden, dtype, seed=rows)


def test_general_tier_forced(abi):
    from hp_rms_norm_amd.abi import Config
    cfg = Config(3, 256, 0, 0, 256, 0, 0)
    for hidden in (8, 4096, 32768):
        check_case(abi, 19, hidden, torch.bfloat16, seed=hidden, config=cfg)


@pytest.mark.parametrize("pad", [3, 8, 24])
def test_strided_and_misaligned_rows(abi, pad):
    """Rows inside a wider buffer (row stride = hidden + pad) and, for odd pads,
    16-byte misaligned row starts; both tensors offset by one element."""
    rows, hidden, eps, dtype = 50, 2048, 1e-6, torch.bfloat16
    x, r, w = make_inputs(rows, hidden, dtype, pad)
    want_out, want_res = oracle_fused(x, r, w, eps, dtype)
    for offset in (0, 1):
        bx = torch.zeros(rows, hidden + pad + offset, dtype=dtype, device=DEV)
        br = torch.zeros(rows, hidden + pad + offset, dtype=dtype, device=DEV)
        xd = bx[:, offset:offset + hidden]
        rd = br[:, offset:offset + hidden]
        xd.copy_(x.to(DEV))
        rd.copy_(r.to(DEV))
        wd = w.to(DEV)
        abi.fused_add_rmsnorm(xd.data_ptr(), wd.data_ptr(), rd.data_ptr(), rows, hidden, xd.stride(0),
                              rd.stride(0), DT[dtype], eps, _stream())
        torch.cuda.synchronize()
        assert_residual_exact(bits(rd), want_res, dtype)
        assert_output_close(bits(xd), want_out, dtype)
        # the padding around the rows is untouched
        assert torch.count_nonzero(bx[:, :offset]) == 0 and torch.count_nonzero(bx[:, offset + hidden:]) == 0
        assert torch.count_nonzero(br[:, offset + hidden:]) == 0


def test_3d_input_and_empty(abi):
    import hp_rms_norm_amd
    x, r, w = make_inputs(6, 4096, torch.bfloat16, 5)
    want_out, want_res = oracle_fused(x, r, w, 1e-6, torch.bfloat16)
    xd = x.to(DEV).view(2, 3, 4096)
    rd = r.to(DEV).view(2, 3, 4096)
    hp_rms_norm_amd.hp_rms_norm(xd, w.to(DEV), rd, 1e-6)
    torch.cuda.synchronize()
    assert_residual_exact(bits(rd), want_res, torch.bfloat16)
    assert_output_close(bits(xd), want_out, torch.bfloat16)
    e = torch.empty(0, 4096, dtype=torch.bfloat16, device=DEV)
    hp_rms_norm_amd.hp_rms_norm(e, w.to(DEV), e.clone(), 1e-6)
    # rows of width 0: every op returns without a launch
    z = lambda *s, dt=torch.bfloat16: torch.empty(*s, dtype=dt, device=DEV)  # noqa: E731
    ops = hp_rms_norm_amd
    ops.hp_rms_norm(z(4, 0), z(0), z(4, 0), 1e-6)
    ops.relu(z(2, 3, 0), z(2, 3, 0))
    ops.rms_norm(z(4, 0), z(4, 0), z(0), 1e-6)
    ops.fused_add_rms_norm_out(z(4, 0), z(4, 0), z(4, 0), z(0), z(4, 0), 1e-6)
    ops.hp_rms_norm_fp8(z(4, 0, dt=torch.float8_e4m3fn), z(4, 1, dt=torch.float32), z(4, 0), z(0), z(4, 0), 1e-6)
    ops.reduce_add_rms_norm(z(4, 0), [z(4, 0)], z(0), z(4, 0), 1e-6)
    ops.hp_rms_norm_mx(z(4, 0, dt=torch.uint8), z(4, 0, dt=torch.uint8), z(4, 0), z(0), z(4, 0), 1e-6, ops.MXFP4)
    torch.cuda.synchronize()


# ---- size-independent properties at the largest configuration ---------------------------
def test_full_size_properties(abi):
    """At (4096, 32768): the residual equals torch's own HIP bf16 add
    bit-for-bit, the output is within 1 ulp of a float32 torch evaluation of
    the reference formula on the GPU, and permuting rows permutes outputs
    bit-for-bit (rows are independent)."""
    import hp_rms_norm_amd
    rows, hidden, eps, dtype = 4096, 32768, 1e-6, torch.bfloat16
    x, r, w = make_inputs(rows, hidden, dtype, 99)
    xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
    s_ref = xd + rd
    sf = s_ref.float()
    o_ref = ((sf * torch.rsqrt(sf.pow(2).mean(-1, keepdim=True) + eps)) * wd.float()).to(dtype)
    perm = torch.randperm(rows, generator=torch.Generator().manual_seed(3)).to(DEV)
    xp, rp = xd[perm].contiguous(), rd[perm].contiguous()
    hp_rms_norm_amd.hp_rms_norm(xd, wd, rd, eps)
    hp_rms_norm_amd.hp_rms_norm(xp, wd, rp, eps)
    torch.cuda.synchronize()
    assert torch.equal(rd.view(torch.int16), s_ref.view(torch.int16))
    assert_output_close(bits(xd), bits(o_ref), dtype)
    assert torch.equal(xp.view(torch.int16), xd[perm].view(torch.int16))
    assert torch.equal(rp.view(torch.int16), rd[perm].view(torch.int16))


def test_batch_beyond_2_pow_31_elements(abi):
    """(2^19 + 5, 4096) bf16: 2.15e9 elements per tensor, so row offsets pass
    2^31 elements.  The whole residual must equal torch's HIP add bit-for-bit
    and the whole output must be within 1 ulp of a float32 torch evaluation
    (checked in row chunks); the first and last rows are also checked against
    the CPU oracle."""
    import hp_rms_norm_amd
    rows, hidden, eps, dtype = (1 << 19) + 5, 4096, 1e-6, torch.bfloat16
    g = torch.Generator(device=DEV).manual_seed(5)
    x = torch.randn((rows, hidden), generator=g, device=DEV, dtype=torch.float32).to(dtype)
    r = torch.randn((rows, hidden), generator=g, device=DEV, dtype=torch.float32).to(dtype)
    w = make_inputs(1, hidden, dtype, 3)[2].to(DEV)
    ends = torch.cat([torch.arange(0, 64), torch.arange(rows - 64, rows)]).to(DEV)
    xe, re_ = x[ends].cpu(), r[ends].cpu()
    s_ref = x + r
    hp_rms_norm_amd.hp_rms_norm(x, w, r, eps)
    torch.cuda.synchronize()
    assert torch.equal(r.view(torch.int16), s_ref.view(torch.int16))
    del s_ref
    wf = w.float()

    def ordered(t):  # bf16 bits on the ordered-integer line (no NaNs occur here)
        i = t.view(torch.int16).to(torch.int32)
        mag = i & 0x7FFF
        return torch.where(i < 0, -mag, mag)

    for c0 in range(0, rows, 65536):
        sf = r[c0:c0 + 65536].float()
        o = ((sf * torch.rsqrt(sf.pow(2).mean(-1, keepdim=True) + eps)) * wf).to(dtype)
        d = int((ordered(x[c0:c0 + 65536]) - ordered(o)).abs().max())
        assert d <= 1, f"rows {c0}..: {d} ulp"
    want_out, want_res = oracle_fused(xe, re_, w.cpu(), eps, dtype)
    assert_residual_exact(bits(r[ends]), want_res, dtype)
    assert_output_close(bits(x[ends]), want_out, dtype)


def test_torch_compile_functionalises_the_in_place_op(abi):
    """torch.compile (aot_eager: no codegen) traces the op through its Meta
    kernel and functionalises its declared in-place writes; the compiled
    function must give the eager result bit-for-bit."""
    import hp_rms_norm_amd

    def f(x, w, r):
        y = x * 2
        hp_rms_norm_amd.hp_rms_norm(y, w, r, 1e-6)
        return y + 0, r + 0

    x, r, w = (t.to(DEV) for t in make_inputs(64, 4096, torch.bfloat16, 21))
    want_y, want_r = f(x.clone(), w, r.clone())
    got_y, got_r = torch.compile(f, backend="aot_eager", fullgraph=True)(x.clone(), w, r.clone())
    torch.cuda.synchronize()
    assert torch.equal(got_y.view(torch.int16), want_y.view(torch.int16))
    assert torch.equal(got_r.view(torch.int16), want_r.view(torch.int16))


def test_torch_compile_with_the_other_ops(abi):
    """The out-of-place, plain, FP8 (per row, static, per group) / MX and partial-sum ops through
    torch.compile (aot_eager, fullgraph): their alias annotations and Meta
    kernels let functionalisation see every write; bit-for-bit equal to eager."""
    import hp_rms_norm_amd as h

    def f(x, w, r, p1, s1):
        out, res = h.fused_add_rms_norm(x, r, w, 1e-6)
        plain = torch.empty_like(x)
        h.rms_norm(plain, x, w, 1e-6)
        r8 = r.clone()
        q8, s8 = h.fused_add_rms_norm_fp8(x, r8, w, 1e-6)
        rs = r.clone()
        qs = h.fused_add_rms_norm_fp8_static(x, rs, w, s1, 1e-6)
        rg = r.clone()
        qg, sg = h.fused_add_rms_norm_fp8_group(x, rg, w, 1e-6)
        r4 = r.clone()
        q4, s4 = h.fused_add_rms_norm_mxfp4(x, r4, w, 1e-6)
        rp, o2 = r.clone(), torch.empty_like(x)
        h.reduce_add_rms_norm(o2, [x, p1], w, rp, 1e-6)
        return (out, res, plain, q8.view(torch.uint8), s8, r8, qs.view(torch.uint8), rs, qg.view(torch.uint8), sg,
                rg, q4.view(torch.uint8), s4.view(torch.uint8), r4, o2, rp)

    x, r, w = (t.to(DEV) for t in make_inputs(96, 2048, torch.bfloat16, 22))
    p1 = torch.randn(96, 2048, device=DEV).to(torch.bfloat16)
    s1 = torch.full((1,), 0.02, device=DEV)
    want = f(x, w, r, p1, s1)
    got = torch.compile(f, backend="aot_eager", fullgraph=True)(x, w, r, p1, s1)
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(got, want)):
        assert a.dtype == b.dtype and a.shape == b.shape, i
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8)), f"output {i} differs"


# ---- streams and graphs ------------------------------------------------------------------
def test_runs_on_current_stream(abi):
    import hp_rms_norm_amd
    x, r, w = make_inputs(512, 8192, torch.bfloat16, 11)
    want_out, want_res = oracle_fused(x, r, w, 1e-6, torch.bfloat16)
    s = torch.cuda.Stream()
    xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        hp_rms_norm_amd.hp_rms_norm(xd, wd, rd, 1e-6)
    s.synchronize()
    assert_residual_exact(bits(rd), want_res, torch.bfloat16)
    assert_output_close(bits(xd), want_out, torch.bfloat16)


def test_concurrent_threads_and_streams(abi):
    """Four host threads, each on its own stream with its own tensors, call
    the op repeatedly; every result matches the oracle."""
    import threading

    import hp_rms_norm_amd
    shapes = [(300, 4096), (17, 8192), (1000, 1024), (64, 32768)]
    data = []
    for i, (rows, hidden) in enumerate(shapes):
        x, r, w = make_inputs(rows, hidden, torch.bfloat16, 600 + i)
        data.append((x, r, w, oracle_fused(x, r, w, 1e-6, torch.bfloat16)))
    results, errors = {}, []

    def worker(i):
        try:
            x, r, w, _ = data[i]
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                for _ in range(5):
                    xd, rd, wd = x.to(DEV, non_blocking=False), r.to(DEV), w.to(DEV)
                    hp_rms_norm_amd.hp_rms_norm(xd, wd, rd, 1e-6)
            s.synchronize()
            results[i] = (bits(xd), bits(rd))
        except Exception as e:  # surfaced below
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(shapes))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for i in range(len(shapes)):
        want_out, want_res = data[i][3]
        assert_residual_exact(results[i][1], want_res, torch.bfloat16)
        assert_output_close(results[i][0], want_out, torch.bfloat16)


def test_hip_graph_capture_and_replay(abi):
    """The op allocates nothing and issues no memset, so it can be captured;
    each replay (fresh inputs copied in between, with eager work and syncs
    around it) must match the eager result."""
    import hp_rms_norm_amd
    rows, hidden, eps, dtype = 256, 4096, 1e-6, torch.bfloat16
    xs = torch.empty(rows, hidden, dtype=dtype, device=DEV)
    rs = torch.empty_like(xs)
    wd = make_inputs(1, hidden, dtype, 0)[2].to(DEV)
    xs.normal_()
    rs.normal_()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        hp_rms_norm_amd.hp_rms_norm(xs, wd, rs, eps)  # warm-up outside the graph
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        hp_rms_norm_amd.hp_rms_norm(xs, wd, rs, eps)
    for rep in range(4):
        x, r, _ = make_inputs(rows, hidden, dtype, 100 + rep)
        xs.copy_(x.to(DEV))
        rs.copy_(r.to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        got_x, got_r = xs.clone(), rs.clone()
        xe, re_ = x.to(DEV), r.to(DEV)
        hp_rms_norm_amd.hp_rms_norm(xe, wd, re_, eps)
        torch.cuda.synchronize()
        assert torch.equal(got_x.view(torch.int16), xe.view(torch.int16)), f"replay {rep} output"
        assert torch.equal(got_r.view(torch.int16), re_.view(torch.int16)), f"replay {rep} residual"


# ---- plain RMSNorm ---------------------------------------------------------------------
@pytest.mark.parametrize("hidden", [128, 1000, 4096, 12288, 32768])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_plain_rmsnorm(abi, hidden, dtype):
    import hp_rms_norm_amd
    x, _, w = make_inputs(33, hidden, dtype, hidden)
    want = oracle.rmsnorm(bits(x), bits(w), 1e-6, DT[dtype], threads=8)
    xd, wd = x.to(DEV), w.to(DEV)
    out = torch.empty_like(xd)
    hp_rms_norm_amd.rms_norm(out, xd, wd, 1e-6)
    torch.cuda.synchronize()
    assert_output_close(bits(out), want, dtype)
    assert torch.equal(xd.cpu().view(torch.int16), x.view(torch.int16))  # input untouched
    hp_rms_norm_amd.rms_norm(xd, xd, wd, 1e-6)                           # in place
    torch.cuda.synchronize()
    assert torch.equal(xd.view(torch.int16), out.view(torch.int16))


@pytest.mark.parametrize("rows,hidden", [(1024, 4096), (2048, 3584), (800, 5120)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_plain_rmsnorm_wave_rows(abi, rows, hidden, dtype):
    """Plain RMSNorm at 3K-5K, 768 < rows <= 2048: one row per one-wave workgroup."""
    import hp_rms_norm_amd
    c = abi.select_config(rows, hidden, DT[dtype], abi.MODE_PLAIN)
    assert (c.lanes_per_row, c.block_threads) == (64, 64), c.as_tuple()
    x, _, w = make_inputs(rows, hidden, dtype, rows + hidden)
    want = oracle.rmsnorm(bits(x), bits(w), 1e-6, DT[dtype], threads=8)
    xd, wd = x.to(DEV), w.to(DEV)
    out = torch.empty_like(xd)
    hp_rms_norm_amd.rms_norm(out, xd, wd, 1e-6)
    torch.cuda.synchronize()
    assert_output_close(bits(out), want, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_plain_rmsnorm_every_table_row(abi, dtype):
    """Enough rows for the bandwidth table (its plain-RMSNorm rows included),
    every row of it with a ragged width, against the oracle."""
    import hp_rms_norm_amd
    for hidden in (128, 256, 512, 1000, 2048, 3064, 4096, 4104, 5120, 6144, 8192, 12288, 16376, 24576, 28672, 32768,
                   65536):
        print("plain", hidden, dtype, flush=True)
        x, _, w = make_inputs(1100, hidden, dtype, hidden + 1)
        want = oracle.rmsnorm(bits(x), bits(w), 1e-6, DT[dtype], threads=min(16, oracle.max_threads()))
        xd, wd = x.to(DEV), w.to(DEV)
        out = torch.empty_like(xd)
        hp_rms_norm_amd.rms_norm(out, xd, wd, 1e-6)
        torch.cuda.synchronize()
        assert_output_close(bits(out), want, dtype, f"plain 1100x{hidden} {dtype}")


@pytest.mark.parametrize("hidden", [13, 1001, 4095, 16383, 20001])
def test_plain_rmsnorm_odd_widths(abi, hidden):
    """Odd widths take the vector tiers' tail variants (the general tier for
    every mode is tested in test_gpu_unaligned.py)."""
    import hp_rms_norm_amd
    for dtype in (torch.bfloat16, torch.float16):
        x, _, w = make_inputs(21, hidden, dtype, hidden)
        want = oracle.rmsnorm(bits(x), bits(w), 1e-6, DT[dtype], threads=min(16, oracle.max_threads()))
        xd, wd = x.to(DEV), w.to(DEV)
        out = torch.empty_like(xd)
        hp_rms_norm_amd.rms_norm(out, xd, wd, 1e-6)
        torch.cuda.synchronize()
        assert_output_close(bits(out), want, dtype, f"plain general 21x{hidden} {dtype}")


def test_functional_form(abi):
    import hp_rms_norm_amd
    x, r, w = make_inputs(64, 4096, torch.bfloat16, 8)
    want_out, want_res = oracle_fused(x, r, w, 1e-6, torch.bfloat16)
    xd, rd = x.to(DEV), r.to(DEV)
    out, res = hp_rms_norm_amd.fused_add_rms_norm(xd, rd, w.to(DEV), 1e-6)
    torch.cuda.synchronize()
    assert_residual_exact(bits(res), want_res, torch.bfloat16)
    assert_output_close(bits(out), want_out, torch.bfloat16)
    assert torch.equal(xd.cpu().view(torch.int16), x.view(torch.int16))
    assert torch.equal(rd.cpu().view(torch.int16), r.view(torch.int16))


# ---- errors raised on the GPU path --------------------------------------------------------
def test_errors_on_device_tensors(abi):
    import hp_rms_norm_amd
    x = torch.zeros(4, 256, dtype=torch.bfloat16, device=DEV)
    w = torch.ones(256, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="input.dim"):
        hp_rms_norm_amd.hp_rms_norm(x[0], w, x[0].clone(), 1e-6)
    with pytest.raises(RuntimeError, match="dtype must be kFloat16 or kBFloat16"):
        hp_rms_norm_amd.hp_rms_norm(x.float(), w.float(), x.float().clone(), 1e-6)
    with pytest.raises(RuntimeError, match="weight.dtype"):
        hp_rms_norm_amd.hp_rms_norm(x, w.half(), x.clone(), 1e-6)
    with pytest.raises(RuntimeError):
        hp_rms_norm_amd.hp_rms_norm(x, w, x, 1e-6)  # input aliases residual
    with pytest.raises(RuntimeError, match="same device"):
        hp_rms_norm_amd.hp_rms_norm(x, w.cpu(), x.clone(), 1e-6)
    xt = torch.zeros(256, 4, dtype=torch.bfloat16, device=DEV).t()   # [4, 256], inner stride 4
    with pytest.raises(RuntimeError, match=r"input.stride\(-1\) == 1"):
        hp_rms_norm_amd.hp_rms_norm(xt, w, x.clone(), 1e-6)


# ---- the per-mode end of the latency rows; small in-place calls without sc1 ------------
@pytest.mark.parametrize("hidden,limit", [(1024, 1024), (2048, 768), (4096, 768), (12288, 384)])
def test_fused_on_both_sides_of_the_latency_row_limit(abi, hidden, limit):
    """The fused op's latency rows end at a per-width row count: the last row
    count that takes them and the first that does not, through the torch op,
    against the oracle."""
    lat = abi.select_config(1, hidden, abi.DTYPE_BF16).as_tuple()
    for rows in (limit, limit + 1):
        assert (abi.select_config(rows, hidden, abi.DTYPE_BF16).as_tuple() == lat) == (rows == limit)
        check_case(abi, rows, hidden, torch.bfloat16, seed=rows, via="torch")


@pytest.mark.parametrize("rows,hidden", [(512, 12288), (1024, 16384), (1536, 9216), (320, 32768)])
def test_small_in_place_calls_without_sc1_give_the_table_kernels_bits(abi, rows, hidden):
    """Calls with rows * hidden <= 2^24 run the table's shape without the sc1
    bits; the bits equal those of the table's kernel (forced, sc1 included),
    and the oracle's bar holds."""
    c = abi.select_config(rows, hidden, abi.DTYPE_BF16)
    assert rows * hidden <= 1 << 24 and c.flags & 24, c.as_tuple()
    x, r, w = make_inputs(rows, hidden, torch.bfloat16, seed=hidden + rows)
    outs = []
    for config in (None, c):
        xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
        run_abi(abi, xd, wd, rd, 1e-6, config)
        torch.cuda.synchronize()
        outs.append((bits(xd), bits(rd)))
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    check_case(abi, rows, hidden, torch.bfloat16, seed=hidden + rows)


# ---- the device's CU count ---------------------------------------------------------------
def test_device_cu_count_is_the_devices(abi):
    """The CU count the entry points size their row rules by is the device's
    own (hipDeviceAttributeMultiprocessorCount, cached per device): torch
    reports the same count, and a call at a row count where the rules depend
    on it gives the bits of the table's choice at that count, forced, and
    meets the oracle's bar."""
    n = abi.device_cu_count(0)
    assert n == torch.cuda.get_device_properties(0).multi_processor_count
    assert abi.device_cu_count(-1) == n and abi.device_cu_count(0) == n   # cached, current device
    rows, hidden = 1280, 2048   # wide rows on 256 CUs
    c = abi.select_config(rows, hidden, abi.DTYPE_BF16, cus=n)
    print("cus", n, "config", c.as_tuple(), flush=True)
    x, r, w = make_inputs(rows, hidden, torch.bfloat16, seed=n)
    outs = []
    for config in (None, c):
        xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
        run_abi(abi, xd, wd, rd, 1e-6, config)
        torch.cuda.synchronize()
        outs.append((bits(xd), bits(rd)))
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    check_case(abi, rows, hidden, torch.bfloat16, seed=n)


# ---- row groups in runs per XCD ------------------------------------------------------------
@pytest.mark.parametrize("rows,hidden", [(4096, 4096), (4100, 4096), (2048, 8192), (4133, 8192), (16384, 8192)])
def test_xcd_runs_rows_give_the_default_orders_bits(abi, rows, hidden):
    """At the row pitches where the in-place op takes its row groups in runs
    per XCD (flags bits 16-18), the bits equal those of the same kernel in
    the default order (forced), also with a partial last block of runs, and
    the oracle's bar holds."""
    c = abi.select_config(rows, hidden, abi.DTYPE_BF16, cus=abi.device_cu_count())
    assert (c.flags >> 16) & 7, c.as_tuple()
    plain = abi.Config(*c.as_tuple())
    plain.flags = c.flags & 0xffff
    x, r, w = make_inputs(rows, hidden, torch.bfloat16, seed=hidden + rows)
    outs = []
    for config in (None, plain):
        xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
        run_abi(abi, xd, wd, rd, 1e-6, config)
        torch.cuda.synchronize()
        outs.append((bits(xd), bits(rd)))
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    check_case(abi, rows, hidden, torch.bfloat16, seed=hidden + rows)
