"""The bench library (libhprms_bench.so) on the GPU: the kernel shapes only
the tuning sweeps use meet the parity bar against the oracle, the timeline
entry point gives the table kernels' results and a well-formed per-workgroup
record, and the ceiling kernels move exactly the bytes they claim.  bench.py
times these kernels beside the product's, so they are held to the same bar."""
import numpy as np
import pytest
import torch

from helpers import DT, assert_output_close, assert_residual_exact, bits, make_inputs, oracle_fused

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def abi():
    assert torch.cuda.is_available(), "the gpu tests need a HIP device"
    import hp_rms_norm_amd  # noqa: F401
    from hp_rms_norm_amd import abi as a
    a.BENCH.lib()
    return a


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _widths(cfg):
    cover = cfg.lanes_per_row * cfg.vec_per_lane * 8
    return sorted({cover, max(8, cover - 8), max(8, cover - cfg.lanes_per_row * 8 + 8)})


def test_bench_only_shapes_meet_the_bar(abi):
    prod = {c.as_tuple() for c in abi.kernel_configs(abi.DTYPE_BF16)}
    extra = [c for c in abi.BENCH.kernel_configs(abi.DTYPE_BF16)
             if c.as_tuple() not in prod and not (c.flags & 512)]
    assert extra
    for cfg in extra:
        rpb = cfg.block_threads // cfg.lanes_per_row
        for hidden in _widths(cfg):
            rows = 3 * rpb + 1
            print("bench config", cfg.as_tuple(), "hidden", hidden, flush=True)
            x, r, w = make_inputs(rows, hidden, torch.bfloat16, seed=hidden + rows)
            want_out, want_res = oracle_fused(x, r, w, 1e-6, torch.bfloat16)
            xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
            abi.BENCH.fused_add_rmsnorm(xd.data_ptr(), wd.data_ptr(), rd.data_ptr(), rows, hidden, hidden, hidden,
                                        abi.DTYPE_BF16, 1e-6, _stream(), cfg)
            torch.cuda.synchronize()
            tag = f"{cfg.as_tuple()} {rows}x{hidden}"
            assert_residual_exact(bits(rd), want_res, torch.bfloat16, "residual " + tag)
            assert_output_close(bits(xd), want_out, torch.bfloat16, "output " + tag)


def test_timeline_entry_point(abi):
    import ctypes
    L = abi.BENCH.lib()
    tl_cfgs = [c for c in abi.BENCH.kernel_configs(abi.DTYPE_BF16) if c.flags & 512]
    assert tl_cfgs
    for cfg in tl_cfgs:
        rpb = cfg.block_threads // cfg.lanes_per_row
        hidden = cfg.lanes_per_row * cfg.vec_per_lane * 8
        rows = 5 * rpb + 1
        grid = (rows + rpb - 1) // rpb
        print("timeline config", cfg.as_tuple(), "hidden", hidden, flush=True)
        x, r, w = make_inputs(rows, hidden, torch.bfloat16, seed=hidden)
        want_out, want_res = oracle_fused(x, r, w, 1e-6, torch.bfloat16)
        xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
        tl = torch.zeros((grid, 4), dtype=torch.int64, device=DEV)
        rc = L.hprms_bench_fused_timeline(xd.data_ptr(), wd.data_ptr(), rd.data_ptr(), rows, hidden,
                                          abi.DTYPE_BF16, 1e-6, ctypes.byref(cfg), tl.data_ptr(), _stream())
        assert rc == 0, abi.BENCH.last_error()
        torch.cuda.synchronize()
        tag = f"{cfg.as_tuple()} {rows}x{hidden}"
        assert_residual_exact(bits(rd), want_res, torch.bfloat16, "residual " + tag)
        assert_output_close(bits(xd), want_out, torch.bfloat16, "output " + tag)
        t = tl.cpu().numpy()
        assert (t[:, 0] > 0).all() and (t[:, 1] >= t[:, 0]).all(), tag
        assert (t[:, 1] - t[:, 0]).max() < 100_000_000, tag    # under a second of 10 ns ticks
        assert ((t[:, 3] & 0xF) < 8).all(), tag                 # XCC ids of the 8 XCDs


def test_ceiling_kernels_move_what_they_claim(abi):
    L = abi.BENCH.lib()
    s = _stream()
    n = 1 << 20                                              # bytes per tensor
    a = torch.randint(0, 2 ** 31 - 1, (n // 4,), dtype=torch.int32, device=DEV)
    b = torch.randint(0, 2 ** 31 - 1, (n // 4,), dtype=torch.int32, device=DEV)
    d = torch.zeros_like(a)
    assert L.hprms_ceil_copy(d.data_ptr(), a.data_ptr(), n, s) == 0
    torch.cuda.synchronize()
    assert torch.equal(d, a)
    sink = torch.zeros(4, dtype=torch.int32, device=DEV)
    assert L.hprms_ceil_read(a.data_ptr(), b.data_ptr(), n, sink.data_ptr(), s) == 0
    wa, wb = torch.zeros_like(a), torch.zeros_like(a)
    assert L.hprms_ceil_write(wa.data_ptr(), wb.data_ptr(), n, s) == 0
    for block in (64, 128, 256, 512, 1024):
        assert L.hprms_ceil_empty(1000, block, s) == 0
    torch.cuda.synchronize()
    v = np.arange(n // 16, dtype=np.uint32).repeat(4)
    assert np.array_equal(wa.cpu().numpy().view(np.uint32), v)
    assert np.array_equal(wb.cpu().numpy().view(np.uint32), ~v)


@pytest.mark.parametrize("shape", [(128, 4, 256, 131), (512, 2, 512, 3), (1024, 4, 1024, 155), (64, 4, 256, 27),
                                   (32, 12, 64, 131), (64, 8, 512, 131), (512, 1, 512, 131), (128, 4, 128, 131)])
def test_skeleton_moves_the_ops_bytes(abi, shape):
    """r <- x + r and x <- x ^ (r_new + t) per 32-bit word, t the binary32 bits of
    the row's sum of the low bytes of r_new's words (exact in fp32 at these sizes)."""
    lpr, vpl, block, flags = shape
    rows, hidden = 3 * (block // lpr) + 1, lpr * vpl * 8 - 8
    g = torch.Generator(device=DEV).manual_seed(lpr)
    x = torch.randint(0, 2 ** 31 - 1, (rows, hidden // 2), dtype=torch.int32, device=DEV, generator=g)
    r = torch.randint(0, 2 ** 31 - 1, (rows, hidden // 2), dtype=torch.int32, device=DEV, generator=g)
    x0, r0 = x.cpu().numpy().view(np.uint32), r.cpu().numpy().view(np.uint32)
    assert abi.BENCH.lib().hprms_ceil_skeleton(x.data_ptr(), r.data_ptr(), rows, hidden, lpr, vpl, block, flags,
                                               _stream()) == 0
    torch.cuda.synchronize()
    s = x0 + r0
    t = np.array([np.float32((row & 0xFF).sum(dtype=np.int64)) for row in s]).view(np.uint32)
    assert np.array_equal(r.cpu().numpy().view(np.uint32), s)
    assert np.array_equal(x.cpu().numpy().view(np.uint32), x0 ^ (s + t[:, None]))



def test_stream_pattern_kernels(abi):
    """hprms_ceil_streams: kind 0 adds 1 to every 32-bit word of a in place;
    kind 1 stores a + b to a and a ^ b to b; kind 2 stores them to c and d."""
    L = abi.BENCH.lib()
    s = _stream()
    n = 1 << 20
    g = torch.Generator(device=DEV).manual_seed(3)
    a = torch.randint(0, 2 ** 31 - 1, (n // 4,), dtype=torch.int32, device=DEV, generator=g)
    b = torch.randint(0, 2 ** 31 - 1, (n // 4,), dtype=torch.int32, device=DEV, generator=g)
    a0, b0 = a.cpu().numpy().view(np.uint32), b.cpu().numpy().view(np.uint32)
    c, d = torch.zeros_like(a), torch.zeros_like(a)
    assert L.hprms_ceil_streams(2, a.data_ptr(), b.data_ptr(), c.data_ptr(), d.data_ptr(), n, s) == 0
    torch.cuda.synchronize()
    assert np.array_equal(c.cpu().numpy().view(np.uint32), a0 + b0)
    assert np.array_equal(d.cpu().numpy().view(np.uint32), a0 ^ b0)
    assert L.hprms_ceil_streams(1, a.data_ptr(), b.data_ptr(), None, None, n, s) == 0
    torch.cuda.synchronize()
    assert np.array_equal(a.cpu().numpy().view(np.uint32), a0 + b0)
    assert np.array_equal(b.cpu().numpy().view(np.uint32), a0 ^ b0)
    ab = torch.cat([a, b])
    ab0 = ab.cpu().numpy().view(np.uint32).copy()
    assert L.hprms_ceil_streams(0, ab.data_ptr(), None, None, None, n, s) == 0
    torch.cuda.synchronize()
    assert np.array_equal(ab.cpu().numpy().view(np.uint32), ab0 + 1)


def test_flat_stream_kernels(abi):
    """hprms_ceil_flat at every built shape and load order, on a size that
    leaves the last workgroup partly past the end: kind 0 adds 1 to every
    32-bit word of a (2n bytes) in place; kind 1 stores a + b to b and
    a ^ b to a."""
    import bench
    L = abi.BENCH.lib()
    s = _stream()
    n = (1 << 20) + 3 * 4096 + 48
    g = torch.Generator(device=DEV).manual_seed(5)
    a0 = torch.randint(0, 2 ** 31 - 1, (n // 4,), dtype=torch.int32, device=DEV, generator=g)
    b0 = torch.randint(0, 2 ** 31 - 1, (n // 4,), dtype=torch.int32, device=DEV, generator=g)
    ua, ub = a0.cpu().numpy().view(np.uint32), b0.cpu().numpy().view(np.uint32)
    for block, vpl in bench.FLAT_SHAPES:
        ab = torch.cat([a0, b0])
        assert L.hprms_ceil_flat(0, block, vpl, 0, ab.data_ptr(), None, n, s) == 0
        torch.cuda.synchronize()
        assert np.array_equal(ab.cpu().numpy().view(np.uint32), np.concatenate([ua, ub]) + 1), (block, vpl)
        for order in range(4):
            print("flat", block, vpl, order, flush=True)
            a, b = a0.clone(), b0.clone()
            assert L.hprms_ceil_flat(1, block, vpl, order, a.data_ptr(), b.data_ptr(), n, s) == 0
            torch.cuda.synchronize()
            assert np.array_equal(b.cpu().numpy().view(np.uint32), ua + ub), (block, vpl, order)
            assert np.array_equal(a.cpu().numpy().view(np.uint32), ua ^ ub), (block, vpl, order)
