"""Pins of the oracle's OCP MX step (oracle/hprms_oracle.c, mx_quantize_row),
on the CPU.  The reference has no block-scaled output; the step is defined by
the OCP Microscaling Formats (MX) v1.0 specification, and these checks fix it
independently of the oracle's code:
  * the E2M1 conversion against a restatement by rounding thresholds (the
    oracle searches for the nearest value), and against hand-worked ties;
  * the E8M0 scale encoding against torch's float8_e8m0fnu conversion;
  * the whole step against a numpy restatement from the specification
    (np.frexp for the block exponent, np.ldexp for the scaling, torch's
    float8_e4m3fn conversion for MXFP8 elements) on blocks spanning the whole
    exponent range, zeros, subnormals, NaN and infinity;
  * closed forms worked by hand;
and every planted mistake of the step is rejected by at least one of them.
The fused MX oracle is the pinned fused oracle followed by this step.
"""
import numpy as np
import pytest
import torch

from oracle import oracle

BF, HF = oracle.BF16, oracle.FP16
TDT = {BF: torch.bfloat16, HF: torch.float16}
E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], np.float32)


def bits16(values, code):
    return torch.tensor(values, dtype=torch.float64).to(TDT[code]).view(torch.int16).numpy().view(np.uint16)


def f32_of(bits, code):
    """16-bit patterns to float32 through numpy / torch conversions only."""
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    if code == HF:
        return b.view(np.float16).astype(np.float32)
    return (b.astype(np.uint32) << 16).view(np.float32)


def e2m1_by_thresholds(v):
    """Round to nearest E2M1 with ties to the even code, from the midpoints of
    the value table (a tie goes to the neighbour whose mantissa bit is 0)."""
    a = np.abs(v)
    code = ((a > 0.25).astype(np.int32) + (a >= 0.75) + (a > 1.25) + (a >= 1.75) + (a > 2.5) + (a >= 3.5)
            + (a > 5.0))
    code = np.where(np.isnan(a), 7, code)    # no NaN code: the largest, with NaN's sign
    return (np.signbit(v).astype(np.uint8) << 3) | code.astype(np.uint8)


def mx_by_spec(y_bits, code, elem):
    """numpy restatement of the MX step from the specification."""
    y = f32_of(y_bits, code)
    rows, hidden = y.shape
    blocks = y.reshape(rows, hidden // 32, 32)
    a = np.abs(blocks)
    bad = np.isnan(a).any(-1) | np.isinf(a).any(-1)
    amax = np.where(bad, 1.0, np.where(np.isnan(a), 0, a).max(-1))
    _, e = np.frexp(amax)
    emax = 8 if elem == oracle.MXFP8 else 2
    s = np.clip(e - 1 - emax, -127, 127)
    s = np.where(amax == 0, -127, s)
    scales = np.where(bad, 255, s + 127).astype(np.uint8)
    v = np.where(bad[..., None], blocks, np.ldexp(blocks, -s[..., None]).astype(np.float32)).astype(np.float32)
    if elem == oracle.MXFP8:
        v = np.clip(v, -448.0, 448.0)
        q = torch.from_numpy(np.ascontiguousarray(v)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        return q.reshape(rows, hidden), scales
    c = e2m1_by_thresholds(v).reshape(rows, hidden)
    return (c[:, 0::2] | (c[:, 1::2] << 4)).astype(np.uint8), scales


def spanning_inputs(code, seed=0, rows=24, hidden=256):
    """Blocks of N(0,1) values scaled by 2^k over the type's whole exponent
    range, plus zero, subnormal, power-of-two, NaN and infinity blocks."""
    rng = np.random.default_rng(seed)
    y = rng.standard_normal((rows, hidden // 32, 32))
    lo, hi = (-140, 125) if code == BF else (-26, 14)
    k = rng.integers(lo, hi, size=(rows, hidden // 32, 1))
    y = y * np.exp2(k.astype(np.float64))
    y[0, 0] = 0.0
    y[0, 1] = 2.0 ** (-135 if code == BF else -24) * rng.integers(1, 4, 32)      # subnormals
    y[0, 2] = 2.0 ** rng.integers(-5, 5, 32)                                        # powers of two
    y[1, 0, 3] = np.nan
    y[1, 1, 7] = -np.inf
    y[1, 2] = 6.0 * np.sign(rng.standard_normal(32))                                 # at the E2M1 maximum
    with np.errstate(over="ignore"):
        return bits16(y.reshape(rows, hidden), code)


def pin_spec(mutation=0):
    for code in (BF, HF):
        for elem in (oracle.MXFP8, oracle.MXFP4):
            y = spanning_inputs(code, seed=code * 2 + elem)
            q, sc = oracle.mx_quantize(y, code, elem, mutation=mutation)
            wq, wsc = mx_by_spec(y, code, elem)
            if not np.array_equal(sc, wsc):
                return f"dtype {code} elem {elem}: scales differ from the specification"
            if elem == oracle.MXFP8:
                nan = (wq & 0x7F) == 0x7F                    # torch encodes NaN as 0x7F, the oracle as 0xFF
                ok = np.array_equal(q[~nan], wq[~nan]) and np.all((q[nan] & 0x7F) == 0x7F)
            else:
                ok = np.array_equal(q, wq)
            if not ok:
                return f"dtype {code} elem {elem}: elements differ from the specification"
    return None


def pin_closed_forms(mutation=0):
    def quant(values, elem, code=BF):
        y = bits16([values], code)
        return oracle.mx_quantize(y, code, elem, mutation=mutation)
    # all ones: floor(log2 1) = 0, so 2^-2 (E2M1: 1 -> 4.0, code 6) and 2^-8 (E4M3: 256 = 0x78)
    q, sc = quant([1.0] * 32, oracle.MXFP4)
    if sc[0, 0] != 125 or not np.all(q == 0x66):
        return "ones, MXFP4"
    q, sc = quant([1.0] * 32, oracle.MXFP8)
    if sc[0, 0] != 119 or not np.all(q == 0x78):
        return "ones, MXFP8"
    # amax 3: floor(log2 3) = 1, scale 2^-1, 3 -> 6.0 (code 7); a ceiling would give 2^0 and 3.0 (code 5)
    q, sc = quant([3.0] * 32, oracle.MXFP4)
    if sc[0, 0] != 126 or not np.all(q == 0x77):
        return "threes, MXFP4"
    # amax 4 (scale 2^0): the ties 0.25 .75 1.25 1.75 2.5 3.5 5 go to codes 0 2 2 4 4 6 6
    vals = [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 4.0] * 4
    q, sc = quant(vals, oracle.MXFP4)
    codes = np.stack([q[0] & 0xF, q[0] >> 4], 1).reshape(-1)
    if sc[0, 0] != 127 or list(codes[:8]) != [0, 2, 2, 4, 4, 6, 6, 6]:
        return "ties, MXFP4"
    # nibble order: element 0 in the low nibble
    q, _ = quant([0.5, 1.0] + [4.0] * 30, oracle.MXFP4)
    if q[0, 0] != 0x21:
        return "nibble order"
    # a zero block takes the smallest scale; a NaN or an infinity marks the block 0xFF
    q, sc = quant([0.0] * 32, oracle.MXFP4)
    if sc[0, 0] != 0 or np.any(q):
        return "zero block"
    for bad in (float("nan"), float("inf")):
        _, sc = quant([1.0] * 31 + [bad], oracle.MXFP8)
        if sc[0, 0] != 255:
            return "NaN / inf block"
    return None


def test_e2m1_conversion_by_thresholds_and_by_hand():
    rng = np.random.default_rng(7)
    v = np.concatenate([rng.standard_normal(200000).astype(np.float32) * 3,
                        np.float32([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0, 7.0, 1e30, np.inf, -np.inf, -0.0,
                                    np.nan]),
                        E2M1, -E2M1, (E2M1[1:] + E2M1[:-1]) / 2])
    assert np.array_equal(oracle.e2m1_from_f32(v), e2m1_by_thresholds(v))
    assert list(oracle.e2m1_from_f32(E2M1)) == list(range(8))                 # every value is its own code
    assert list(oracle.e2m1_from_f32(np.float32([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0]))) == [0, 2, 2, 4, 4, 6, 6]


def test_e8m0_encoding_matches_torch():
    s = np.arange(-127, 128)
    want = torch.from_numpy(np.exp2(s.astype(np.float64)).astype(np.float32)).to(torch.float8_e8m0fnu)
    assert np.array_equal(want.view(torch.uint8).numpy(), (s + 127).astype(np.uint8))
    for k in (-127, -3, 0, 5, 120):   # blocks whose maximum is exactly 2^(k + emax) get the byte k + 127
        _, sc = oracle.mx_quantize(bits16([[2.0 ** (k + 2)] * 32], BF), BF, oracle.MXFP4)
        assert sc[0, 0] == k + 127


def test_mx_step_matches_the_specification():
    assert pin_spec() is None


def test_mx_closed_forms():
    assert pin_closed_forms() is None


@pytest.mark.parametrize("name", sorted(oracle.MX_MUTATIONS))
def test_planted_mx_mistake_is_rejected(name):
    m = oracle.MX_MUTATIONS[name]
    assert [f for f in (pin_spec(m), pin_closed_forms(m)) if f], f"no pin rejects {name!r}"


@pytest.mark.parametrize("elem", [oracle.MXFP8, oracle.MXFP4], ids=["mxfp8", "mxfp4"])
@pytest.mark.parametrize("code", [BF, HF], ids=["bf16", "fp16"])
def test_fused_mx_oracle_is_the_fused_op_then_the_mx_step(code, elem):
    g = torch.Generator().manual_seed(3)
    x, r = (torch.randn(40, 512, generator=g).to(TDT[code]) for _ in range(2))
    w = (1 + 0.1 * torch.randn(512, generator=g)).to(TDT[code])
    xb, rb, wb = (t.view(torch.int16).numpy().view(np.uint16) for t in (x, r, w))
    q, sc, res = oracle.fused_add_rmsnorm_mx(xb, wb, rb, 1e-6, code, elem)
    y, res2 = oracle.fused_add_rmsnorm(xb, wb, rb, 1e-6, code)
    wq, wsc = oracle.mx_quantize(y, code, elem)
    assert np.array_equal(res, res2) and np.array_equal(q, wq) and np.array_equal(sc, wsc)
