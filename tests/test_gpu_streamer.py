"""GPU parity of the streamer: the reference's "relu" (an identity copy,
activation_kernels.cuh:99-119, pinned by test/test_relu.py:24) and the true
ReLU beside it, against the CPU oracle and torch.relu.  Bit-exact."""
import random

import numpy as np
import pytest
import torch

from helpers import DT, bits, from_bits
from oracle import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def ops():
    assert torch.cuda.is_available(), "the gpu tests need a HIP device"
    import hp_rms_norm_amd
    return hp_rms_norm_amd


def _rand(rows, hidden, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn((rows, hidden), generator=g).to(dtype)


def test_golden_streamer(ops, golden):
    for name, c in golden.items():
        if c["kind"] != "stream":
            continue
        dtype = torch.bfloat16 if c["dtype"] == "bf16" else torch.float16
        x = from_bits(c["x"], dtype).to(DEV)
        out = torch.full_like(x, 7.0)
        ops.relu(out, x)
        torch.cuda.synchronize()
        assert np.array_equal(bits(out), c["copy"]), name
        ops.relu_max0(out, x)
        torch.cuda.synchronize()
        d = oracle.ulp_distance(bits(out), c["relu"], DT[dtype])  # NaN payloads may differ from torch's
        assert d.max() == 0, name


def test_reference_relu_sweep(ops):
    """test/test_relu.py:27-33: H = 128 ... 32768 step 128 with random token
    counts, out must equal inp; here seeded, both dtypes."""
    rng = random.Random(77)
    for dtype in (torch.bfloat16, torch.float16):
        for hidden in range(128, 32768 + 128, 128):
            rows = rng.randint(1, 48)
            x = (0.1 * _rand(rows, hidden, torch.float32, hidden)).to(dtype).to(DEV)
            out = torch.zeros_like(x)
            ops.relu(out, x)
            torch.cuda.synchronize()
            assert torch.equal(out.view(torch.int16), x.view(torch.int16)), (rows, hidden, dtype)


@pytest.mark.parametrize("rows,hidden", [(4096, 14336), (1, 1), (3, 13), (7, 1000), (129, 4104)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_streamer_vs_oracle(ops, rows, hidden, dtype):
    x = _rand(rows, hidden, dtype, rows + hidden)
    x.view(-1)[: min(6, x.numel())] = torch.tensor([0.0, -0.0, float("nan"), -float("inf"), -1e-30, 2.0])[
        : min(6, x.numel())].to(dtype)
    xd = x.to(DEV)
    for op, fn in ((oracle.COPY, ops.relu), (oracle.RELU, ops.relu_max0)):
        out = torch.empty_like(xd)
        fn(out, xd)
        torch.cuda.synchronize()
        want = oracle.streamer(bits(x), DT[dtype], op)
        assert np.array_equal(bits(out), want), (op, rows, hidden)
    # torch.relu on the GPU also agrees in value; it differs only in the sign
    # of zero (HIP torch.relu(-0.0) is +0.0, CPU torch.relu keeps -0.0, as this
    # kernel and the oracle do), which a value comparison ignores.
    out = torch.empty_like(xd)
    ops.relu_max0(out, xd)
    torch.testing.assert_close(out, torch.relu(xd), rtol=0, atol=0, equal_nan=True)


# the row kernel (strided or misaligned rows): H < 8 (one element per lane), odd widths (the
# tail vector), one 4 KiB chunk exactly (2048) and one vector past it, several chunks
STRIDED_WIDTHS = [1, 7, 8, 9, 1000, 1001, 2048, 2049, 2056, 14337, 40000]


@pytest.mark.parametrize("hidden", STRIDED_WIDTHS)
def test_streamer_strided_and_misaligned(ops, hidden):
    for dtype in (torch.bfloat16, torch.float16):
        for offset, pad in ((0, 8), (1, 3), (1, 0), (3, 5)):
            rows = 31
            x = _rand(rows, hidden, dtype, hidden + offset)
            for name, fn, op in (("copy", ops.relu, oracle.COPY), ("relu", ops.relu_max0, oracle.RELU)):
                print("streamer rows", hidden, dtype, offset, pad, name, flush=True)
                bi = torch.zeros(rows, hidden + pad + offset, dtype=dtype, device=DEV)
                bo = torch.zeros_like(bi)
                xi = bi[:, offset:offset + hidden]
                xo = bo[:, offset + 1:offset + 1 + hidden] if pad else bo[:, offset:offset + hidden]
                xi.copy_(x.to(DEV))
                fn(xo, xi)
                torch.cuda.synchronize()
                want = oracle.streamer(bits(x), DT[dtype], op)
                assert np.array_equal(bits(xo), want), (hidden, offset, pad, name)
                lo = offset + 1 if pad else offset
                assert torch.count_nonzero(bo[:, :lo]) == 0 and torch.count_nonzero(bo[:, lo + hidden:]) == 0
                # in place on the strided view
                fn(xi, xi)
                torch.cuda.synchronize()
                assert np.array_equal(bits(xi), want), ("in place", hidden, offset, pad, name)


def test_streamer_in_place(ops):
    x = _rand(64, 4096, torch.bfloat16, 9)
    xd = x.to(DEV)
    ops.relu_max0(xd, xd)
    torch.cuda.synchronize()
    assert np.array_equal(bits(xd), oracle.streamer(bits(x), oracle.BF16, oracle.RELU))
