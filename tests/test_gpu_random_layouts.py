"""GPU parity over seeded random layouts, every mode against the oracle.

Each case draws a dtype, a width (1 ... 70000, weighted towards the table's
boundaries and odd values), a row count, and for every stream its own element
offset into a wider buffer and its own row padding; so the streams of one call
can start at different 2-byte boundaries with different strides (every third
case puts all streams at one offset and padding, which the shifted rows need),
and the dispatch picks among the aligned kernels, their unaligned and tail
variants and the general tier.  Bar as everywhere: residual bit-exact, 16-bit output within
1 ulp, FP8 within one step, MX scales and elements bit-exact against the
oracle's MX step of the same kernel family's 16-bit output.  The cases are
fixed by the seed, so a failure names a reproducible layout.
"""
import random

import numpy as np
import pytest
import torch

from helpers import DT, assert_output_close, assert_residual_exact, bits, lane_mapping, make_inputs, oracle_fused
from oracle import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
EPS = 1e-6
TABLE_EDGES = [128, 256, 512, 1024, 2048, 3072, 4096, 8192, 12288, 16376, 16384, 24576, 32768, 65536]


@pytest.fixture(scope="module")
def abi():
    assert torch.cuda.is_available(), "the gpu tests need a HIP device"
    import hp_rms_norm_amd  # noqa: F401
    from hp_rms_norm_amd import abi as a
    a.lib()
    return a


def _stream():
    return torch.cuda.current_stream().cuda_stream


def draw_width(rng):
    kind = rng.random()
    if kind < 0.4:
        return max(1, rng.choice(TABLE_EDGES) + rng.randint(-9, 9))
    if kind < 0.8:
        return rng.randint(1, 70000)
    return rng.randint(1, 600)


def place(t, off, pad):
    """t [rows, hidden] copied into a zero [rows, off + hidden + pad] buffer at
    column `off`; returns (view, buffer)."""
    rows, hidden = t.shape
    buf = torch.zeros(rows, off + hidden + pad, dtype=t.dtype, device=DEV)
    v = buf[:, off:off + hidden]
    v.copy_(t.to(DEV))
    return v, buf


def stride(v):
    return v.stride(0)


def cases(n, seed):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        hidden = draw_width(rng)
        rows = rng.choice([1, 3, 17, 64, 300])
        if hidden > 20000:
            rows = min(rows, 17)
        dtype = rng.choice([torch.bfloat16, torch.float16])
        offs = [rng.choice([0, 0, 1, 3, 8, 13]) for _ in range(6)]
        pads = [rng.choice([0, 0, 1, 5, 8, 64]) for _ in range(6)]
        if i % 3 == 2:
            # every stream at one offset and padding: the written streams share one phase,
            # so from 4104 elements up the rows are shifted
            offs, pads = [offs[0]] * 6, [pads[0]] * 6
        out.append((i, hidden, rows, dtype, offs, pads))
    return out


def tag(c):
    i, hidden, rows, dtype, offs, pads = c
    return f"case {i}: {rows}x{hidden} {dtype} offsets {offs} pads {pads}"


@pytest.mark.parametrize("case", cases(40, 1234), ids=lambda c: f"c{c[0]}-h{c[1]}")
def test_random_layouts_fused_plain_out(abi, case):
    i, hidden, rows, dtype, offs, pads = case
    t = tag(case)
    print(t, flush=True)
    x, r, w = make_inputs(rows, hidden, dtype, seed=i + 100)
    want_out, want_res = oracle_fused(x, r, w, EPS, dtype)
    wv, _ = place(w[None], offs[5] % 2, 0)
    # in place
    xv, xb = place(x, offs[0], pads[0])
    rv, rb = place(r, offs[1], pads[1])
    abi.fused_add_rmsnorm(xv.data_ptr(), wv.data_ptr(), rv.data_ptr(), rows, hidden, stride(xv), stride(rv), DT[dtype],
                          EPS, _stream())
    torch.cuda.synchronize()
    assert_residual_exact(bits(rv), want_res, dtype, "fused residual " + t)
    assert_output_close(bits(xv), want_out, dtype, "fused output " + t)
    for b, off, h in ((xb, offs[0], hidden), (rb, offs[1], hidden)):
        assert not bits(b[:, :off]).any() and not bits(b[:, off + h:]).any(), "wrote outside the rows " + t
    # out of place
    xv, _ = place(x, offs[0], pads[0])
    rv, _ = place(r, offs[1], pads[1])
    ov, ob = place(torch.zeros_like(x), offs[2], pads[2])
    rov, rob = place(torch.zeros_like(x), offs[3], pads[3])
    abi.fused_add_rmsnorm_out(ov.data_ptr(), rov.data_ptr(), xv.data_ptr(), rv.data_ptr(), wv.data_ptr(), rows,
                              hidden, stride(ov), stride(rov), stride(xv), stride(rv), DT[dtype], EPS, _stream())
    torch.cuda.synchronize()
    assert_residual_exact(bits(rov), want_res, dtype, "out residual " + t)
    assert_output_close(bits(ov), want_out, dtype, "out output " + t)
    assert np.array_equal(bits(xv), bits(x)) and np.array_equal(bits(rv), bits(r)), "out: inputs modified " + t
    for b, off in ((ob, offs[2]), (rob, offs[3])):
        assert not bits(b[:, :off]).any() and not bits(b[:, off + hidden:]).any(), "wrote outside the rows " + t
    # plain RMSNorm
    ov, ob = place(torch.zeros_like(x), offs[4], pads[4])
    abi.rmsnorm(ov.data_ptr(), xv.data_ptr(), wv.data_ptr(), rows, hidden, stride(ov), stride(xv), DT[dtype], EPS,
                _stream())
    torch.cuda.synchronize()
    want = oracle.rmsnorm(bits(x), bits(w), EPS, DT[dtype], threads=min(16, oracle.max_threads()))
    assert_output_close(bits(ov), want, dtype, "plain " + t)
    assert not bits(ob[:, :offs[4]]).any() and not bits(ob[:, offs[4] + hidden:]).any(), "wrote outside " + t


@pytest.mark.parametrize("case", cases(30, 4321), ids=lambda c: f"c{c[0]}-h{c[1]}")
def test_random_layouts_fp8_and_reduce(abi, case):
    i, hidden, rows, dtype, offs, pads = case
    t = tag(case)
    print(t, flush=True)
    x, r, w = make_inputs(rows, hidden, dtype, seed=i + 200)
    wv, _ = place(w[None], offs[5] % 2, 0)
    threads = min(16, oracle.max_threads())
    # FP8 output: q rows at any byte offset
    xv, _ = place(x, offs[0], pads[0])
    rv, _ = place(r, offs[1], pads[1])
    qb = torch.zeros(rows, offs[2] + hidden + pads[2], dtype=torch.uint8, device=DEV)
    q = qb[:, offs[2]:offs[2] + hidden]
    sc = torch.empty(rows, dtype=torch.float32, device=DEV)
    abi.fused_add_rmsnorm_fp8(q.data_ptr(), sc.data_ptr(), xv.data_ptr(), wv.data_ptr(), rv.data_ptr(), rows, hidden,
                              qb.stride(0), stride(xv), stride(rv), DT[dtype], EPS, _stream())
    torch.cuda.synchronize()
    oq, osc, ores = oracle.fused_add_rmsnorm_fp8(bits(x), bits(w), bits(r), EPS, DT[dtype], threads=threads)
    assert_residual_exact(bits(rv), ores, dtype, "fp8 residual " + t)
    assert oracle.e4m3_ulp_distance(q.contiguous().cpu().numpy(), oq).max() <= 1, "fp8 " + t
    np.testing.assert_allclose(sc.cpu().numpy(), osc, rtol=2.0 ** -7, err_msg="fp8 scale " + t)
    assert not qb[:, :offs[2]].any() and not qb[:, offs[2] + hidden:].any(), "fp8 wrote outside " + t
    # partial sums: 1-4 parts sharing one row stride, each at its own offset
    g = random.Random(i)
    nparts = g.randint(1, 4)
    gen = torch.Generator().manual_seed(i + 300)
    parts = [torch.randn((rows, hidden), generator=gen).to(dtype) for _ in range(nparts)]
    pstride = hidden + 8 + pads[3]
    pbuf = torch.zeros(nparts, rows, pstride + 8, dtype=dtype, device=DEV)
    poffs = [g.choice([0, 1, 3, 8]) for _ in range(nparts)]
    pviews = [pbuf[k, :, poffs[k]:poffs[k] + hidden] for k in range(nparts)]
    for pv, p in zip(pviews, parts):
        pv.copy_(p.to(DEV))
    rv, _ = place(r, offs[1], pads[1])
    ov, ob = place(torch.zeros_like(x), offs[4], pads[4])
    abi.reduce_add_rmsnorm(ov.data_ptr(), [p.data_ptr() for p in pviews], wv.data_ptr(), rv.data_ptr(), rows, hidden,
                           stride(ov), pbuf.shape[2], stride(rv), DT[dtype], EPS, _stream())
    torch.cuda.synchronize()
    p_out, p_res = oracle.reduce_add_rmsnorm([bits(p) for p in parts], bits(w), bits(r), EPS, DT[dtype],
                                             threads=threads)
    assert_residual_exact(bits(rv), p_res, dtype, f"reduce residual ({nparts} parts) " + t)
    assert_output_close(bits(ov), p_out, dtype, f"reduce output ({nparts} parts) " + t)
    assert not bits(ob[:, :offs[4]]).any() and not bits(ob[:, offs[4] + hidden:]).any(), "wrote outside " + t


# widths 32 ... 65536 (the MX outputs have no general-tier fallback above the table)
@pytest.mark.parametrize("case", [c for c in cases(60, 777) if 32 <= c[1] - c[1] % 32 <= 65536][:24],
                         ids=lambda c: f"c{c[0]}-h{c[1]}")
def test_random_layouts_mx(abi, case):
    """MX outputs (hidden rounded down to a multiple of 32): scales and elements
    equal the oracle's MX step of the 16-bit output the same table shape
    produces in place on contiguous copies (the same lane mapping)."""
    i, hidden, rows, dtype, offs, pads = case
    hidden -= hidden % 32
    t = tag(case) + f" (hidden {hidden})"
    print(t, flush=True)
    x, r, w = make_inputs(rows, hidden, dtype, seed=i + 400)
    for fmt, elem in ((abi.MX_FP8_E4M3, oracle.MXFP8), (abi.MX_FP4_E2M1, oracle.MXFP4)):
        qw = hidden if fmt == abi.MX_FP8_E4M3 else hidden // 2
        xv, _ = place(x, offs[0], pads[0])
        rv, _ = place(r, offs[1], pads[1])
        wv, _ = place(w[None], offs[5] % 2, 0)
        qb = torch.zeros(rows, offs[2] + qw + pads[2], dtype=torch.uint8, device=DEV)
        sb = torch.zeros(rows, offs[3] + hidden // 32 + pads[3], dtype=torch.uint8, device=DEV)
        q, s = qb[:, offs[2]:offs[2] + qw], sb[:, offs[3]:offs[3] + hidden // 32]
        abi.fused_add_rmsnorm_mx(q.data_ptr(), s.data_ptr(), xv.data_ptr(), wv.data_ptr(), rv.data_ptr(), rows, hidden,
                                 qb.stride(0), sb.stride(0), stride(xv), stride(rv), fmt, DT[dtype], EPS, _stream())
        # the 16-bit output of the same shape (in place, contiguous copies)
        mode = abi.MODE_MXFP8 if fmt == abi.MX_FP8_E4M3 else abi.MODE_MXFP4
        cfg = lane_mapping(abi, abi.select_config(rows, hidden, DT[dtype], mode))
        y, r16, wd = x.to(DEV), r.to(DEV), w.to(DEV)
        abi.BENCH.fused_add_rmsnorm(y.data_ptr(), wd.data_ptr(), r16.data_ptr(), rows, hidden, hidden, hidden, DT[dtype],
                                    EPS, _stream(), cfg)
        torch.cuda.synchronize()
        assert np.array_equal(bits(rv), bits(r16)), "mx residual " + t
        wq, wsc = oracle.mx_quantize(bits(y).reshape(rows, hidden), DT[dtype], elem)
        sn = s.contiguous().cpu().numpy()
        qn = q.contiguous().cpu().numpy()
        assert np.array_equal(sn, wsc), "mx scales " + t
        per = 32 if elem == oracle.MXFP8 else 16
        live = (wsc != 0xFF)
        assert np.all((qn.reshape(rows, -1, per) == wq.reshape(rows, -1, per)).all(-1) | ~live), "mx elements " + t
        assert not qb[:, :offs[2]].any() and not qb[:, offs[2] + qw:].any(), "mx wrote outside " + t
        assert not sb[:, :offs[3]].any() and not sb[:, offs[3] + hidden // 32:].any(), "mx scales outside " + t
