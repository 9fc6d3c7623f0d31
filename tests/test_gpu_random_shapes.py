"""GPU parity over seeded random shapes, layouts, modes and data, against the
oracle: row counts up to 6000 (so the table's row-count rules -- latency,
wide, one- and two-wave rows, runs per XCD, the staged weight -- meet random
widths and layouts), widths 1 ... 70000 weighted towards the table's
boundaries, each stream at its own element offset and row padding (or all at
one), every entry point (in place, plain, FP8, out of place, partial sums,
MXFP8, MXFP4), eps in {0, 1e-6, 1e-5, 2^-7}, and the benchmark, outlier,
reference-test and special-value data (tests/helpers.py).

Bar as everywhere: residual bit-exact, 16-bit output within 1 ulp, FP8 the
quantisation of a y within one 16-bit ulp of the oracle's output (the scale
that of an amax within one ulp of the oracle's), MX scales and live elements
bit-exact against the oracle's MX step of the same kernel family's 16-bit
output, and nothing written outside the rows.  The cases are fixed by the seed; each is
printed before it runs, so a failure names a reproducible case.
"""
import math
import random

import numpy as np
import pytest
import torch

from helpers import (DT, assert_fp8_from_y_within_one_ulp, assert_group_scales, assert_output_close,
                     assert_residual_exact, bits, lane_mapping, make_inputs, oracle_fused, special_inputs,
                     special_weight)
from oracle import oracle

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
EDGES = [128, 256, 512, 1024, 1536, 2048, 2560, 3072, 3584, 4096, 5120, 6144, 8192, 12288, 16376, 16384, 20480,
         24576, 32768, 65536]


def draw(rng):
    k = rng.random()
    if k < 0.45:
        hidden = max(1, rng.choice(EDGES) + rng.choice([0, 0, 0, -8, 8, -1, 1, rng.randint(-40, 40)]))
    elif k < 0.85:
        hidden = int(math.exp(rng.uniform(math.log(8), math.log(70000))))
    else:
        hidden = rng.randint(1, 700)
    rows = int(math.exp(rng.uniform(0, math.log(6000))))
    if rng.random() < 0.3:
        rows = rng.choice([256, 384, 385, 512, 513, 768, 769, 1024, 1025, 1280, 1281, 1536, 2048, 2049, 3072,
                           4096, 4097, 5120])
    rows = max(1, min(rows, 12_000_000 // max(hidden, 1)))
    dtype = rng.choice([torch.bfloat16, torch.float16])
    if rng.random() < 0.5:
        offs, pads = [0] * 6, [0] * 6
    else:
        offs = [rng.choice([0, 0, 1, 3, 8, 13, 64]) for _ in range(6)]
        pads = [rng.choice([0, 0, 1, 5, 8, 64, 120]) for _ in range(6)]
        if rng.random() < 0.4:
            offs, pads = [offs[0]] * 6, [pads[0]] * 6
    mode = rng.choice([0, 0, 0, 1, 3, 4, 2, 5, 6])
    if mode in (5, 6):
        hidden = max(32, min(65536, hidden - hidden % 32))
        rows = max(1, min(rows, 12_000_000 // hidden))
    eps = rng.choice([1e-6, 1e-6, 1e-5, 2.0 ** -7, 0.0])
    dist = rng.choice(["bench", "bench", "outliers", "reference_test", "special", "special_weight"])
    return dict(hidden=hidden, rows=rows, dtype=dtype, offs=offs, pads=pads, mode=mode, eps=eps, dist=dist)


def place(t, off, pad):
    rows, hidden = t.shape
    buf = torch.zeros(rows, off + hidden + pad, dtype=t.dtype, device=DEV)
    v = buf[:, off:off + hidden]
    v.copy_(t.to(DEV))
    return v, buf


def outside_clean(buf, off, hidden):
    return not bits(buf[:, :off]).any() and not bits(buf[:, off + hidden:]).any()


def run_case(abi, i, c):
    rows, hidden, dtype, offs, pads, mode, eps = (c[k] for k in ("rows", "hidden", "dtype", "offs", "pads", "mode",
                                                                  "eps"))
    if c["dist"] in ("special", "special_weight"):
        x, r, w = special_inputs(rows, hidden, dtype, seed=i)
        if c["dist"] == "special_weight":
            w = special_weight(w)
    else:
        x, r, w = make_inputs(rows, hidden, dtype, seed=i, dist=c["dist"])
    st = torch.cuda.current_stream().cuda_stream
    wv, _ = place(w[None], offs[5] % 2, 0)
    code = DT[dtype]
    t = f"case {i}: {c}"
    if mode == 0:
        want_out, want_res = oracle_fused(x, r, w, eps, dtype)
        xv, xb = place(x, offs[0], pads[0])
        rv, rb = place(r, offs[1], pads[1])
        abi.fused_add_rmsnorm(xv.data_ptr(), wv.data_ptr(), rv.data_ptr(), rows, hidden, xv.stride(0), rv.stride(0),
                              code, eps, st)
        torch.cuda.synchronize()
        assert_residual_exact(bits(rv), want_res, dtype, "residual " + t)
        assert_output_close(bits(xv), want_out, dtype, "output " + t)
        assert outside_clean(xb, offs[0], hidden) and outside_clean(rb, offs[1], hidden), "outside " + t
    elif mode == 3:
        want_out, want_res = oracle_fused(x, r, w, eps, dtype)
        xv, _ = place(x, offs[0], pads[0])
        rv, _ = place(r, offs[1], pads[1])
        ov, ob = place(torch.zeros_like(x), offs[2], pads[2])
        rov, rob = place(torch.zeros_like(x), offs[3], pads[3])
        abi.fused_add_rmsnorm_out(ov.data_ptr(), rov.data_ptr(), xv.data_ptr(), rv.data_ptr(), wv.data_ptr(), rows,
                                  hidden, ov.stride(0), rov.stride(0), xv.stride(0), rv.stride(0), code, eps, st)
        torch.cuda.synchronize()
        assert_residual_exact(bits(rov), want_res, dtype, "out residual " + t)
        assert_output_close(bits(ov), want_out, dtype, "out output " + t)
        assert outside_clean(ob, offs[2], hidden) and outside_clean(rob, offs[3], hidden), "outside " + t
        assert np.array_equal(bits(xv), bits(x)) and np.array_equal(bits(rv), bits(r)), "inputs modified " + t
    elif mode == 1:
        want = oracle.rmsnorm(bits(x), bits(w), eps, code, threads=16)
        xv, _ = place(x, offs[0], pads[0])
        ov, ob = place(torch.zeros_like(x), offs[4], pads[4])
        abi.rmsnorm(ov.data_ptr(), xv.data_ptr(), wv.data_ptr(), rows, hidden, ov.stride(0), xv.stride(0), code, eps,
                    st)
        torch.cuda.synchronize()
        assert_output_close(bits(ov), want, dtype, "plain " + t)
        assert outside_clean(ob, offs[4], hidden), "outside " + t
    elif mode == 2:
        xv, _ = place(x, offs[0], pads[0])
        rv, _ = place(r, offs[1], pads[1])
        qb = torch.zeros(rows, offs[2] + hidden + pads[2], dtype=torch.uint8, device=DEV)
        q = qb[:, offs[2]:offs[2] + hidden]
        sc = torch.empty(rows, dtype=torch.float32, device=DEV)
        abi.fused_add_rmsnorm_fp8(q.data_ptr(), sc.data_ptr(), xv.data_ptr(), wv.data_ptr(), rv.data_ptr(), rows,
                                  hidden, qb.stride(0), xv.stride(0), rv.stride(0), code, eps, st)
        torch.cuda.synchronize()
        oy, ores = oracle.fused_add_rmsnorm(bits(x), bits(w), bits(r), eps, code, threads=16)
        assert_residual_exact(bits(rv), ores, dtype, "fp8 residual " + t)
        scales = sc.reshape(-1, 1).cpu().numpy()
        assert_group_scales(scales, oy, hidden, dtype, "fp8 scale " + t)
        with np.errstate(divide="ignore"):
            assert_fp8_from_y_within_one_ulp(q.contiguous().cpu().numpy(), oy, np.float32(1.0) / scales, dtype,
                                             "fp8 " + t)
        assert not qb[:, :offs[2]].any() and not qb[:, offs[2] + hidden:].any(), "fp8 outside " + t
    elif mode in (5, 6):
        fmt, elem = (abi.MX_FP8_E4M3, oracle.MXFP8) if mode == 5 else (abi.MX_FP4_E2M1, oracle.MXFP4)
        qw = hidden if mode == 5 else hidden // 2
        xv, _ = place(x, offs[0], pads[0])
        rv, _ = place(r, offs[1], pads[1])
        qb = torch.zeros(rows, offs[2] + qw + pads[2], dtype=torch.uint8, device=DEV)
        sb = torch.zeros(rows, offs[3] + hidden // 32 + pads[3], dtype=torch.uint8, device=DEV)
        q, s_ = qb[:, offs[2]:offs[2] + qw], sb[:, offs[3]:offs[3] + hidden // 32]
        abi.fused_add_rmsnorm_mx(q.data_ptr(), s_.data_ptr(), xv.data_ptr(), wv.data_ptr(), rv.data_ptr(), rows,
                                 hidden, qb.stride(0), sb.stride(0), xv.stride(0), rv.stride(0), fmt, code, eps, st)
        cfg = lane_mapping(abi, abi.select_config(rows, hidden, code,
                                                  abi.MODE_MXFP8 if mode == 5 else abi.MODE_MXFP4))
        y, r16, wd = x.to(DEV), r.to(DEV), w.to(DEV)
        abi.BENCH.fused_add_rmsnorm(y.data_ptr(), wd.data_ptr(), r16.data_ptr(), rows, hidden, hidden, hidden, code,
                                    eps, st, cfg)
        torch.cuda.synchronize()
        want_out, want_res = oracle_fused(x, r, w, eps, dtype)
        assert_residual_exact(bits(rv), want_res, dtype, "mx residual " + t)
        assert_output_close(bits(y), want_out, dtype, "mx 16-bit output " + t)
        wq, wsc = oracle.mx_quantize(bits(y).reshape(rows, hidden), code, elem)
        sn, qn = s_.contiguous().cpu().numpy(), q.contiguous().cpu().numpy()
        assert np.array_equal(sn, wsc), "mx scales " + t
        per = 32 if elem == oracle.MXFP8 else 16
        live = wsc != 0xFF
        assert np.all((qn.reshape(rows, -1, per) == wq.reshape(rows, -1, per)).all(-1) | ~live), "mx elements " + t
        assert not qb[:, :offs[2]].any() and not qb[:, offs[2] + qw:].any(), "mx outside " + t
        assert not sb[:, :offs[3]].any() and not sb[:, offs[3] + hidden // 32:].any(), "mx scales outside " + t
    else:
        g = random.Random(i)
        nparts = g.randint(1, 4)
        gen = torch.Generator().manual_seed(i + 7)
        parts = [x] + [torch.randn((rows, hidden), generator=gen).to(dtype) for _ in range(nparts - 1)]
        pstride = hidden + pads[3]
        pbuf = torch.zeros(nparts, rows, pstride + 16, dtype=dtype, device=DEV)
        poffs = [g.choice([0, 1, 3, 8]) for _ in range(nparts)]
        pviews = [pbuf[k, :, poffs[k]:poffs[k] + hidden] for k in range(nparts)]
        for pv, p in zip(pviews, parts):
            pv.copy_(p.to(DEV))
        rv, _ = place(r, offs[1], pads[1])
        ov, ob = place(torch.zeros_like(x), offs[4], pads[4])
        abi.reduce_add_rmsnorm(ov.data_ptr(), [p.data_ptr() for p in pviews], wv.data_ptr(), rv.data_ptr(), rows,
                               hidden, ov.stride(0), pbuf.shape[2], rv.stride(0), code, eps, st)
        torch.cuda.synchronize()
        p_out, p_res = oracle.reduce_add_rmsnorm([bits(p) for p in parts], bits(w), bits(r), eps, code, threads=16)
        assert_residual_exact(bits(rv), p_res, dtype, "reduce residual " + t)
        assert_output_close(bits(ov), p_out, dtype, "reduce output " + t)
        assert outside_clean(ob, offs[4], hidden), "outside " + t


@pytest.fixture(scope="module")
def abi():
    assert torch.cuda.is_available(), "the gpu tests need a HIP device"
    import hp_rms_norm_amd  # noqa: F401  (registers the torch ops; fails loudly if unbuilt)
    from hp_rms_norm_amd import abi as a
    a.lib()
    return a


SEED, NCASES, CHUNK = 3, 400, 40


def _chunk(k):
    rng = random.Random(SEED)
    drawn = [draw(rng) for _ in range(NCASES)]
    return [(i, drawn[i]) for i in range(k * CHUNK, (k + 1) * CHUNK)]


@pytest.mark.parametrize("chunk", range(NCASES // CHUNK))
def test_random_shapes_and_layouts(abi, chunk):
    for i, c in _chunk(chunk):
        print(f"case {SEED}:{i} {c}", flush=True)
        run_case(abi, SEED * 100000 + i, c)
