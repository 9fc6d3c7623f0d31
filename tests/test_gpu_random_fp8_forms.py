"""Seeded random shapes and layouts for the FP8 outputs with one given scale
(static) and with a scale per 128 elements (per group), through the C ABI,
against the CPU oracle: the residual bit-exact, q the quantisation of a y
within one 16-bit ulp of the oracle's output, the per-group scales those of a
group maximum within one ulp of the oracle's, the bytes around every written
region untouched.  Widths cover the table's rows (any width for the static
form, multiples of 128 for the per-group form, whose scales are rows or
columns), row counts from 1 to a few
thousand, row strides and offsets that move rows off the 16- and 128-byte
grids, both dtypes, eps 0 and 1e-6, and rows of special values.  Each case is
printed before it runs.
"""
import math
import random

import numpy as np
import pytest
import torch

from helpers import (DT, assert_fp8_from_y_within_one_ulp, assert_group_scales, assert_residual_exact, bits,
                     make_inputs, special_inputs)
from oracle import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
SEED, NCASES = 5, 120


@pytest.fixture(scope="module")
def abi():
    assert torch.cuda.is_available(), "the gpu tests need a HIP device"
    import hp_rms_norm_amd  # noqa: F401  (registers the torch ops; fails loudly if unbuilt)
    from hp_rms_norm_amd import abi as a
    a.lib()
    return a


def draw(rng):
    form = rng.choice(["static", "group"])
    if form == "group":
        hidden = 128 * (rng.choice([1, 2, 4, 5, 8, 9, 16, 24, 32, 40, 64, 96, 128, 192, 256, 512])
                        if rng.random() < 0.6 else rng.randint(1, 512))
    else:
        hidden = rng.choice([rng.randint(1, 600), int(math.exp(rng.uniform(math.log(8), math.log(70000)))),
                             rng.choice([1024, 4096, 5120, 8192, 16384, 32768]) + rng.choice([0, 0, 8, -8, 1])])
    rows = max(1, min(int(math.exp(rng.uniform(0, math.log(5000)))), 8_000_000 // max(hidden, 1)))
    aligned = rng.random() < 0.5
    offs = [0, 0, 0, 0] if aligned else [rng.choice([0, 1, 3, 8, 64]) for _ in range(4)]
    pads = [0, 0, 0, 0] if aligned else [rng.choice([0, 1, 8, 120]) for _ in range(4)]
    return dict(form=form, hidden=hidden, rows=rows, dtype=rng.choice([torch.bfloat16, torch.float16]),
                offs=offs, pads=pads, eps=rng.choice([1e-6, 1e-6, 0.0]), special=rng.random() < 0.2,
                scale=rng.choice([0.01, 0.03, 1.0, 2.0 ** -20]))


def place(t, off, pad, dtype=None):
    rows, hidden = t.shape
    buf = torch.zeros(rows, off + hidden + pad, dtype=dtype or t.dtype, device=DEV)
    v = buf[:, off:off + hidden]
    v.copy_(t.to(DEV))
    return v, buf


def run_case(abi, i, c):
    rows, hidden, dtype, offs, pads, eps = (c[k] for k in ("rows", "hidden", "dtype", "offs", "pads", "eps"))
    if c["special"]:
        x, r, w = special_inputs(rows, hidden, dtype, seed=i)
    else:
        x, r, w = make_inputs(rows, hidden, dtype, seed=i)
    code = DT[dtype]
    oy, ores = oracle.fused_add_rmsnorm(bits(x), bits(w), bits(r), eps, code, threads=min(16, oracle.max_threads()))
    st = torch.cuda.current_stream().cuda_stream
    xv, _ = place(x, offs[0], pads[0])
    rv, _ = place(r, offs[1], pads[1])
    wd = w.to(DEV)
    qb = torch.zeros(rows, offs[2] + hidden + pads[2], dtype=torch.uint8, device=DEV)
    q = qb[:, offs[2]:offs[2] + hidden]
    t = f"case {i}: {c}"
    if c["form"] == "static":
        sd = torch.tensor([c["scale"]], dtype=torch.float32, device=DEV)
        abi.fused_add_rmsnorm_fp8_static(q.data_ptr(), sd.data_ptr(), xv.data_ptr(), wd.data_ptr(), rv.data_ptr(),
                                         rows, hidden, qb.stride(0), xv.stride(0), rv.stride(0), code, eps, st)
        torch.cuda.synchronize()
        with np.errstate(divide="ignore", over="ignore"):
            isc = np.float32(1.0) / np.float32(c["scale"])
    else:
        ng = hidden // 128
        colmajor = random.Random(i).random() < 0.4
        if colmajor:
            # column-major scales: [groups, rows + pad] with the rows at an offset
            t += " (column-major scales)"
            sb = torch.full((ng, offs[3] + rows + pads[3]), -1.0, dtype=torch.float32, device=DEV)
            sv = sb[:, offs[3]:offs[3] + rows].t()
        else:
            sb = torch.full((rows, offs[3] + ng + pads[3]), -1.0, dtype=torch.float32, device=DEV)
            sv = sb[:, offs[3]:offs[3] + ng]
        abi.fused_add_rmsnorm_fp8_group(q.data_ptr(), sv.data_ptr(), xv.data_ptr(), wd.data_ptr(), rv.data_ptr(),
                                        rows, hidden, qb.stride(0), sv.stride(0), sv.stride(1), xv.stride(0),
                                        rv.stride(0), code, eps, st)
        torch.cuda.synchronize()
        scales = sv.cpu().numpy()
        assert_group_scales(scales, oy, 128, dtype, "scales " + t)
        with np.errstate(divide="ignore"):
            isc = np.repeat(np.float32(1.0) / scales, 128, axis=1)
        written = torch.zeros_like(sb, dtype=torch.bool)
        (written[:, offs[3]:offs[3] + rows] if colmajor else written[:, offs[3]:offs[3] + ng]).fill_(True)
        assert (sb[~written] == -1.0).all(), "scales outside " + t
    assert_residual_exact(bits(rv), ores, dtype, "residual " + t)
    assert np.array_equal(bits(xv), bits(x)), "input modified " + t
    assert_fp8_from_y_within_one_ulp(q.contiguous().cpu().numpy(), oy, isc, dtype, "q " + t)
    assert not qb[:, :offs[2]].any() and not qb[:, offs[2] + hidden:].any(), "q outside " + t


CHUNK = 30


@pytest.mark.parametrize("chunk", range(NCASES // CHUNK))
def test_random_fp8_forms(abi, chunk):
    rng = random.Random(SEED)
    drawn = [draw(rng) for _ in range(NCASES)]
    for i in range(chunk * CHUNK, (chunk + 1) * CHUNK):
        print(f"case {SEED}:{i} {drawn[i]}", flush=True)
        run_case(abi, SEED * 100000 + i, drawn[i])
