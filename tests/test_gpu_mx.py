"""GPU parity of the fused add+RMSNorm with an OCP MX output (MXFP8 / MXFP4).

Pins: the residual is bit-exact against the oracle; the scales and elements
equal, bit for bit, the oracle's MX step (pinned in tests/test_oracle_mx.py)
applied to the 16-bit output the same kernel family produces for the same
inputs (the 16-bit op run with the MX kernel's lane mapping, hence the same
reduction order); against the oracle end to end, every block whose 16-bit
values match the oracle's is bit-exact.  Blocks marked NaN (scale 0xFF) are
compared by their scale only: their element bits are not part of the format.
`input` is not modified.
"""
import numpy as np
import pytest
import torch

from helpers import DT, assert_residual_exact, bits, lane_mapping, make_inputs
from oracle import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
FMT = {"mxfp8": oracle.MXFP8, "mxfp4": oracle.MXFP4}


@pytest.fixture(scope="module")
def ops():
    assert torch.cuda.is_available(), "the gpu tests need a HIP device"
    import hp_rms_norm_amd
    return hp_rms_norm_amd


def u8(t):
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


def compare_blocks(q, sc, wq, wsc, hidden, elem, tag, only=None):
    """q/sc against wq/wsc; `only` masks the blocks to compare ([rows, H/32])."""
    rows = sc.shape[0]
    per = 32 if elem == oracle.MXFP8 else 16
    qb = q.reshape(rows, hidden // 32, per)
    wqb = wq.reshape(rows, hidden // 32, per)
    mask = np.ones(sc.shape, bool) if only is None else only
    assert np.array_equal(sc[mask], wsc[mask]), f"scales differ: {tag}"
    live = mask & (wsc != 0xFF)
    bad = np.argwhere(live & np.any(qb != wqb, axis=-1))
    assert bad.size == 0, f"elements differ in {len(bad)} blocks, first {bad[0].tolist()}: {tag}"


def run_case(ops, rows, hidden, dtype, elem, seed, dist="bench", eps=1e-6, w=None, x=None, r=None):
    from hp_rms_norm_amd import abi
    x0, r0, w0 = make_inputs(rows, hidden, dtype, seed, dist)
    x = x0 if x is None else x
    r = r0 if r is None else r
    w = w0 if w is None else w
    xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
    fn = ops.fused_add_rms_norm_mxfp8 if elem == oracle.MXFP8 else ops.fused_add_rms_norm_mxfp4
    q, sc = fn(xd, rd, wd, eps)
    cfg = lane_mapping(abi, abi.select_config(rows, hidden, DT[dtype], 5 if elem == oracle.MXFP8 else 6))
    y, r16 = x.to(DEV), r.to(DEV)
    abi.BENCH.fused_add_rmsnorm(y.data_ptr(), wd.data_ptr(), r16.data_ptr(), rows, hidden, hidden, hidden, DT[dtype],
                                eps, torch.cuda.current_stream().cuda_stream, cfg)
    torch.cuda.synchronize()
    tag = f"{rows}x{hidden} {dtype} elem {elem} seed {seed} cfg {cfg.as_tuple()}"
    assert torch.equal(xd.cpu().view(torch.int16), x.view(torch.int16)), "input modified " + tag
    assert torch.equal(rd.view(torch.int16), r16.view(torch.int16)), "residual differs from the 16-bit op " + tag
    qn, scn = u8(q).reshape(rows, -1), u8(sc).reshape(rows, -1)
    # the MX step on the kernel family's own 16-bit output: bit for bit
    wq, wsc = oracle.mx_quantize(bits(y).reshape(rows, hidden), DT[dtype], elem)
    compare_blocks(qn, scn, wq, wsc, hidden, elem, "against the MX step of y: " + tag)
    # end to end against the oracle
    oq, osc, ores = oracle.fused_add_rmsnorm_mx(bits(x), bits(w), bits(r), eps, DT[dtype], elem,
                                                threads=min(16, oracle.max_threads()))
    assert_residual_exact(bits(rd), ores, dtype, "residual " + tag)
    oy, _ = oracle.fused_add_rmsnorm(bits(x), bits(w), bits(r), eps, DT[dtype], threads=min(16, oracle.max_threads()))
    same = np.all(oracle.ulp_distance(bits(y).reshape(rows, hidden), oy, DT[dtype]).reshape(rows, hidden // 32, 32)
                  == 0, axis=-1)
    assert same.mean() > 0.95, tag
    compare_blocks(qn, scn, oq, osc, hidden, elem, "against the oracle: " + tag, only=same)
    return qn, scn


# every row of the table, each with a ragged width below it (hidden % 32 == 0)
HIDDENS = [32, 96, 256, 512, 1024, 1056, 2016, 3072, 4096, 4128, 5120, 8192, 12288, 13312, 16384, 24576, 32768,
           65536]


@pytest.mark.parametrize("fmt", sorted(FMT))
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_mx_every_table_row(ops, dtype, fmt):
    for rows in (1100, 64):
        for hidden in HIDDENS:
            print("mx", fmt, rows, hidden, dtype, flush=True)
            run_case(ops, rows, hidden, dtype, FMT[fmt], seed=rows + hidden)


@pytest.mark.parametrize("fmt", sorted(FMT))
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_mx_blocks_across_the_exponent_range(ops, dtype, fmt):
    """Weights of 2^k per block carry the blocks over the type's exponent
    range (bf16 down to 2^-125, so the E8M0 clamp at 2^-127 is reached),
    with outlier inputs."""
    rows, hidden = 256, 4096
    g = torch.Generator().manual_seed(11)
    lo, hi = (-125, 100) if dtype == torch.bfloat16 else (-16, 10)
    k = torch.randint(lo, hi, (hidden // 32,), generator=g)
    if dtype == torch.bfloat16:
        k[0], k[1] = -130, 120           # a subnormal-weight block (the clamp) and a near-maximum one
    k = k.repeat_interleave(32)
    w = (torch.exp2(k.double()) * (1 + 0.1 * torch.randn(hidden, generator=g, dtype=torch.float64))).to(dtype)
    print("mx range", fmt, dtype, flush=True)
    _, sc = run_case(ops, rows, hidden, dtype, FMT[fmt], seed=5, dist="outliers", w=w)
    if dtype == torch.bfloat16:
        # 2^120-weight blocks: floor(log2 max) is about 119, so the byte is about 119 - emax + 127
        assert np.all(sc[:, 0] == 0) and sc[:, 1].min() >= (230 if fmt == "mxfp8" else 236)


@pytest.mark.parametrize("fmt", sorted(FMT))
def test_mx_zero_nan_and_huge_rows(ops, fmt):
    rows, hidden, dtype = 8, 1024, torch.bfloat16
    x, r, w = make_inputs(rows, hidden, dtype, 3)
    x[0] = 0
    r[0] = 0                                   # y = 0: every block gets the smallest scale
    x[1, 77] = float("nan")                    # the whole row turns NaN: every block 0xFF
    x[2] = x[2] * 1e15                         # large values, normalised back to O(1)
    print("mx special", fmt, flush=True)
    q, sc = run_case(ops, rows, hidden, dtype, FMT[fmt], seed=3, x=x, r=r, w=w)
    assert np.all(sc[0] == 0) and not np.any(q[0]) and np.all(sc[1] == 0xFF)


def test_mx_through_the_c_abi_with_strided_outputs(ops):
    """Row strides in bytes on both outputs (padding left untouched)."""
    from hp_rms_norm_amd import abi
    rows, hidden, dtype = 100, 2048, torch.float16
    x, r, w = make_inputs(rows, hidden, dtype, 9)
    xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
    qbuf = torch.full((rows, hidden // 2 + 64), 0xAB, dtype=torch.uint8, device=DEV)
    sbuf = torch.full((rows, hidden // 32 + 5), 0xCD, dtype=torch.uint8, device=DEV)
    abi.fused_add_rmsnorm_mx(qbuf.data_ptr(), sbuf.data_ptr(), xd.data_ptr(), wd.data_ptr(), rd.data_ptr(), rows,
                             hidden, qbuf.stride(0), sbuf.stride(0), hidden, hidden, abi.MX_FP4_E2M1, DT[dtype], 1e-6,
                             torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    oq, osc, ores = oracle.fused_add_rmsnorm_mx(bits(x), bits(w), bits(r), 1e-6, DT[dtype], oracle.MXFP4,
                                                threads=min(16, oracle.max_threads()))
    assert_residual_exact(bits(rd), ores, dtype)
    qn, sn = u8(qbuf), u8(sbuf)
    assert np.all(qn[:, hidden // 2:] == 0xAB) and np.all(sn[:, hidden // 32:] == 0xCD), "wrote into the padding"
    oy, _ = oracle.fused_add_rmsnorm(bits(x), bits(w), bits(r), 1e-6, DT[dtype])
    y, r16 = x.to(DEV), r.to(DEV)
    ops.hp_rms_norm(y, wd, r16, 1e-6)
    torch.cuda.synchronize()
    same = np.all(oracle.ulp_distance(bits(y).reshape(rows, hidden), oy, DT[dtype]).reshape(rows, -1, 32) == 0, -1)
    compare_blocks(qn[:, :hidden // 2], sn[:, :hidden // 32], oq, osc, hidden, oracle.MXFP4, "strided", only=same)


def test_mx_dequantises_close_to_the_16_bit_output(ops):
    """A size-independent property at the benchmark's size: q * 2^s is within
    half a quantum of y (E2M1 quanta are 0.5 / 1 / 2 at 2^s scale), except
    where y / 2^s lies in (6, 8) and saturates to 6."""
    from hp_rms_norm_amd import abi
    rows, hidden = 4096, 8192
    x, r, w = (t.to(DEV) for t in make_inputs(rows, hidden, torch.bfloat16, 21))
    # y from the 16-bit op with the MX kernel's lane mapping (the same reduction order)
    cfg = lane_mapping(abi, abi.select_config(rows, hidden, abi.DTYPE_BF16, abi.MODE_MXFP4))
    y, r16 = x.clone(), r.clone()
    abi.BENCH.fused_add_rmsnorm(y.data_ptr(), w.data_ptr(), r16.data_ptr(), rows, hidden, hidden, hidden, abi.DTYPE_BF16,
                                1e-6, torch.cuda.current_stream().cuda_stream, cfg)
    q, sc = ops.fused_add_rms_norm_mxfp4(x, r, w, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(r.view(torch.int16), r16.view(torch.int16))
    codes = q.view(torch.uint8)
    c = torch.stack([codes & 0xF, codes >> 4], -1).reshape(rows, hidden).long()
    table = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], device=DEV)
    val = table[c & 7] * torch.where(c >= 8, -1.0, 1.0)
    s = sc.view(torch.uint8).float() - 127.0
    deq = (val.reshape(rows, -1, 32) * torch.exp2(s)[..., None]).reshape(rows, hidden)
    yf = y.float()
    quantum = torch.exp2(s)[..., None].expand(rows, hidden // 32, 32).reshape(rows, hidden)
    v = yf.abs() / quantum
    step = torch.where(v < 2, 0.5, torch.where(v < 4, 1.0, 2.0))
    allowed = torch.where(v > 6, v - 6, step / 2) * quantum
    assert torch.all((deq - yf).abs() <= allowed * (1 + 2 ** -20))
    assert (v > 6).float().mean() < 0.2      # saturation stays the exception
