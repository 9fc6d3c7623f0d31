"""Shared helpers of the test suite: seeded inputs of the benchmark
distributions, bit views and the parity assertions (residual bit-exact,
output within 1 ulp and atol/rtol 1e-2 of the oracle)."""
import numpy as np
import torch

from oracle import oracle

DT = {torch.bfloat16: oracle.BF16, torch.float16: oracle.FP16}
# Tolerance of the normalised output against the oracle (the target's bar):
# at most 1 unit in the last place, and assert_close(atol=1e-2, rtol=1e-2).
MAX_ULP = 1
ATOL = RTOL = 1e-2


def bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(dtype)


def make_inputs(rows, hidden, dtype, seed, dist="bench"):
    """input, residual ~ N(0,1), weight ~ N(1, 0.1) (dist "bench"); "outliers"
    scales a seeded 1% of input entries by 50; "reference_test" is the
    reference test's N(0, 0.1) for all three (test/test_hp_rms_norm.py:29-31)."""
    g = torch.Generator().manual_seed(seed)
    if dist == "reference_test":
        x = torch.normal(0, 0.1, (rows, hidden), generator=g)
        r = torch.normal(0, 0.1, (rows, hidden), generator=g)
        w = torch.normal(0, 0.1, (hidden,), generator=g)
    else:
        x = torch.randn((rows, hidden), generator=g)
        r = torch.randn((rows, hidden), generator=g)
        w = 1 + 0.1 * torch.randn((hidden,), generator=g)
        if dist == "outliers":
            m = torch.rand((rows, hidden), generator=g) < 0.01
            x = torch.where(m, x * 50, x)
    return x.to(dtype), r.to(dtype), w.to(dtype)


# Rows of special values, one pattern per row (row i takes pattern i % len):
# where the sum of squares is infinite the inverse is 0 and finite elements
# give +-0; zero rows with eps = 0 give 0 * inf = NaN; subnormal sums are
# exact in binary32, so their rows are as well defined as normal ones.
SPECIAL_PATTERNS = (
    "normal",            # N(0, 1) row, the control
    "zeros",             # x = r = 0
    "nan",               # one NaN in x
    "inf",               # one +inf in x: the row's sum of squares is +inf
    "inf_minus_inf",     # x = +inf, r = -inf at one element: a NaN sum
    "one_huge",          # one element whose square overflows binary32 (fp16: 60000)
    "sum_overflows",     # every square finite, their binary32 sum infinite (fp16: 60000s)
    "large_finite",      # a sum of squares near a quarter of FLT_MAX (fp16: 200s)
    "subnormal",         # bf16 subnormals 1e-39 (fp16: 1e-7), r = 0
    "squares_subnormal", # 1e-20: the squares are binary32 subnormals (fp16: 1e-4)
    "sum_is_inf",        # x + r overflows the 16-bit type at one element
    "cancels",           # x = -r everywhere: a zero row from large values
    "negative_zeros",    # x = r = -0
    "half_subnormal",    # the first half subnormal, the rest N(0, 1)
)


def special_inputs(rows, hidden, dtype, seed):
    """input, residual, weight (CPU, `dtype`) whose row i holds
    SPECIAL_PATTERNS[i % len] on top of an N(0, 1) row; the special element
    of the one-element patterns moves with the row (the last element for
    rows = 2 mod 3)."""
    bf = dtype == torch.bfloat16
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((rows, hidden), generator=g)
    r = torch.randn((rows, hidden), generator=g)
    w = 1 + 0.1 * torch.randn((hidden,), generator=g)
    inf, nan = float("inf"), float("nan")
    safe = (3.4e38 / (4 * hidden)) ** 0.5
    for i in range(rows):
        p = SPECIAL_PATTERNS[i % len(SPECIAL_PATTERNS)]
        j = hidden - 1 if i % 3 == 2 else (i * 37) % hidden
        if p == "zeros":
            x[i], r[i] = 0.0, 0.0
        elif p == "nan":
            x[i, j] = nan
        elif p == "inf":
            x[i, j] = inf
        elif p == "inf_minus_inf":
            x[i, j], r[i, j] = inf, -inf
        elif p == "one_huge":
            x[i, j], r[i, j] = (1e20 if bf else 6e4), 0.0
        elif p == "sum_overflows":
            x[i], r[i] = (3e18 if bf else 6e4), 0.0
        elif p == "large_finite":
            x[i], r[i] = (safe if bf else 200.0), 0.0
        elif p == "subnormal":
            x[i], r[i] = (1e-39 if bf else 1e-7), 0.0
        elif p == "squares_subnormal":
            x[i], r[i] = (1e-20 if bf else 1e-4), 0.0
        elif p == "sum_is_inf":
            x[i, j] = r[i, j] = 3e38 if bf else 6e4
        elif p == "cancels":
            x[i] = (1e30 if bf else 3e4) * torch.sign(x[i])
            r[i] = -x[i]
        elif p == "negative_zeros":
            x[i], r[i] = -0.0, -0.0
        elif p == "half_subnormal":
            x[i, : hidden // 2], r[i, : hidden // 2] = (1e-39 if bf else 1e-7), 0.0
    return x.to(dtype), r.to(dtype), w.to(dtype)


def special_weight(w):
    """`w` with zeros, a negative zero, infinities, a NaN, a subnormal and the
    largest finite magnitudes at spread-out elements (element 11 * k + 3)."""
    bf = w.dtype == torch.bfloat16
    big = 3e38 if bf else 6e4
    vals = (0.0, -0.0, float("inf"), -float("inf"), float("nan"), 1e-39 if bf else 1e-7, big, -big)
    wf = w.float()
    for k, v in enumerate(vals):
        wf[(11 * k + 3) % w.numel()] = v
    return wf.to(w.dtype)


def oracle_fused(x, r, w, eps, dtype, threads=None):
    if threads is None:
        threads = min(16, oracle.max_threads())
    return oracle.fused_add_rmsnorm(bits(x).reshape(-1, x.shape[-1]), bits(w), bits(r).reshape(-1, x.shape[-1]),
                                    eps, DT[dtype], threads=threads)


def assert_residual_exact(got_bits, want_bits, dtype, what="residual"):
    got = np.asarray(got_bits).reshape(-1)
    want = np.asarray(want_bits).reshape(-1)
    d = oracle.ulp_distance(got, want, DT[dtype])   # NaN vs NaN counts as equal
    bad = np.nonzero((got != want) & (d != 0))[0]
    assert bad.size == 0, (f"{what} not bit-exact at {bad.size} elements; first index {bad[0]}: "
                           f"got 0x{got[bad[0]]:04x} want 0x{want[bad[0]]:04x}")


def assert_output_close(got_bits, want_bits, dtype, what="output"):
    got = np.asarray(got_bits).reshape(-1)
    want = np.asarray(want_bits).reshape(-1)
    d = oracle.ulp_distance(got, want, DT[dtype])
    worst = int(d.max()) if d.size else 0
    assert worst <= MAX_ULP, f"{what}: {int((d > MAX_ULP).sum())} elements beyond {MAX_ULP} ulp (max {worst})"
    gt = from_bits(got, dtype).float()
    wt = from_bits(want, dtype).float()
    torch.testing.assert_close(gt, wt, atol=ATOL, rtol=RTOL, equal_nan=True)
    return d


def as_dispatched(abi, cfg, hidden):
    """`cfg`, a table configuration, as the dispatch runs it on contiguous rows
    of `hidden` elements: rows off the 128-byte grid (hidden * 2 % 128 != 0)
    take its unaligned variant (flags bit 5 set, the sc1 bits cleared: they do
    not change results), which rotates each row's lane mapping by the row's
    phase modulo 512 bytes, and so sums the squares in another order than the
    table's kernel forced on them."""
    if cfg.tier == 3 or hidden % 8 != 0 or (hidden * 2) % 128 == 0:
        return cfg
    c = abi.Config(*cfg.as_tuple())
    c.flags = (c.flags & ~24) | 32
    return c


# ---- FP8 outputs against the oracle's 16-bit output ----------------------------------------
# The 16-bit output y is held to one ulp of the oracle's; an FP8 output quantises the kernel's
# own y, so against the oracle it is pinned as "the quantisation of some y within one ulp of the
# oracle's", element by element.  (One ulp of a subnormal y is a factor of two, which a group's
# or a row's small scale turns into several FP8 steps; a fixed step bound would not hold there.)
def ulp_neighbours(a):
    """(below, a, above): each 16-bit pattern and its neighbours one ulp down
    and up on the ordered line (-0 taken as +0)."""
    a = np.asarray(a, np.uint16).astype(np.int32)
    mag = a & 0x7FFF
    o = np.where((a & 0x8000) != 0, -mag, mag)

    def back(v):
        return np.where(v >= 0, v, 0x8000 | (-v)).astype(np.uint16)
    return back(o - 1), a.astype(np.uint16), back(o + 1)


def _e4m3_of(y_bits, isc, dtype):
    with np.errstate(invalid="ignore", over="ignore"):
        v = oracle.to_f32(y_bits, DT[dtype]) * np.asarray(isc, np.float32)
        v = np.where(v > 448.0, np.float32(448.0), np.where(v < -448.0, np.float32(-448.0), v)).astype(np.float32)
    return oracle.e4m3_from_f32(v)


def assert_fp8_from_y_within_one_ulp(q, y_oracle, isc, dtype, what="q"):
    """q (e4m3fn bytes, shaped like y_oracle) equals e4m3fn(clamp(y * isc)) for
    y one of y_oracle's 16-bit neighbours or itself, at every element; `isc`
    (the reciprocal of the kernel's scale) broadcasts against y_oracle."""
    y = np.asarray(y_oracle, np.uint16)
    q = np.asarray(q, np.uint8).reshape(y.shape)
    isc = np.broadcast_to(np.asarray(isc, np.float32), y.shape)
    # the oracle's own y first; only the elements it does not explain try its neighbours
    idx = np.nonzero(oracle.e4m3_ulp_distance(q, _e4m3_of(y, isc, dtype)) != 0)
    if idx[0].size == 0:
        return
    yi, qi, ii = y[idx], q[idx], isc[idx]
    ok = np.zeros(qi.shape, bool)
    for yc in ulp_neighbours(yi):
        ok |= oracle.e4m3_ulp_distance(qi, _e4m3_of(yc, ii, dtype)) == 0
    bad = np.nonzero(~ok)[0]
    assert bad.size == 0, (f"{what}: {bad.size} elements are no quantisation of a y within 1 ulp; first at "
                           f"{tuple(int(v[bad[0]]) for v in idx)}")


def assert_group_scales(scales, y_oracle, group, dtype, what="scales"):
    """Each scale is max(amax / 448, FLT_MIN) for an amax within one ulp of the
    largest |y| of the oracle's group of `group` elements (a kernel's y within
    one ulp of the oracle's moves the maximum by at most that), NaN where the
    group holds NaN."""
    y = np.asarray(y_oracle, np.uint16)
    rows = y.shape[0]
    mag = (y & 0x7FFF).reshape(rows, -1, group).max(axis=-1)        # NaN patterns order above inf
    tiny = np.float32(np.finfo(np.float32).tiny)
    got = np.asarray(scales, np.float32).reshape(mag.shape)
    ok = np.zeros(mag.shape, bool)
    for m in ulp_neighbours(mag):
        with np.errstate(invalid="ignore"):
            sc = (oracle.to_f32(m & 0x7FFF, DT[dtype]) / np.float32(448.0)).astype(np.float32)
            sc = np.where(sc < tiny, tiny, sc).astype(np.float32)
        ok |= (got.view(np.uint32) == sc.view(np.uint32)) | (np.isnan(got) & np.isnan(sc))
    bad = np.argwhere(~ok)
    assert bad.size == 0, f"{what}: {len(bad)} scales off; first {bad[0]}: {got[tuple(bad[0])]}"


def lane_mapping(abi, cfg):
    """`cfg` without the row-order bits (xcd_xor, bit 10; runs per XCD, bits
    16-18): the same lanes, vectors and flags, so the same result for every
    row, with the row groups in the default order.  The 16-bit op that tests
    run with a quantised form's configuration has no run variants of the
    quantised forms' shapes."""
    if cfg is None or cfg.tier == 3:
        return cfg
    c = abi.Config(*cfg.as_tuple())
    c.flags &= ~(1024 | (7 << 16))
    return c
