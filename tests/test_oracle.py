"""Pins of the CPU oracle (oracle/hprms_oracle.c), on the CPU.

Each check is independent of the oracle's own code:
  * golden vectors written by the reference's test formula in torch
    (tests/golden/, test/test_hp_rms_norm.py:6-19 and test/test_relu.py:24),
  * the same formula evaluated live by torch at other shapes,
  * a binary64 brute force written with numpy's own reductions,
  * closed forms: constant rows of powers of two with eps = 0 give +-w
    exactly; scaling a row by a power of two leaves the output unchanged,
  * the 16-bit conversions against numpy's binary16 and torch's bfloat16
    conversions on exhaustive and random bit patterns,
  * rows of special values (NaN, infinities, zero rows with eps = 0, binary32
    overflow of the squares and of their sum, subnormals) against torch,
and every planted mistake the oracle can be asked to make is rejected by at
least one of these pins.
"""
import numpy as np
import pytest
import torch

from helpers import SPECIAL_PATTERNS, special_inputs, special_weight
from oracle import oracle

BF, HF = oracle.BF16, oracle.FP16
TDT = {BF: torch.bfloat16, HF: torch.float16}


def tbits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def tfrom(a, code):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(TDT[code])


def seeded(rows, hidden, code, seed, dist="bench"):
    g = torch.Generator().manual_seed(seed)
    if dist == "reference_test":
        x, r, w = (torch.normal(0, 0.1, s, generator=g) for s in ((rows, hidden), (rows, hidden), (hidden,)))
    else:
        x = torch.randn((rows, hidden), generator=g)
        r = torch.randn((rows, hidden), generator=g)
        w = 1 + 0.1 * torch.randn((hidden,), generator=g)
    dt = TDT[code]
    return tbits(x.to(dt)), tbits(r.to(dt)), tbits(w.to(dt))


def torch_formula(x, r, w, eps, code):
    """The reference test's oracle (test/test_hp_rms_norm.py:6-19), run by torch."""
    xt, rt, wt = tfrom(x, code), tfrom(r, code), tfrom(w, code)
    s = xt + rt
    out = torch.rms_norm(s, normalized_shape=(xt.shape[-1],), weight=wt, eps=eps)
    return tbits(out), tbits(s)


def to_16(v64, code):
    """binary64 -> 16-bit pattern, through numpy / torch conversions only."""
    if code == HF:
        return v64.astype(np.float16).view(np.uint16)   # binary64 -> binary16 directly, RNE
    return tbits(torch.from_numpy(v64).to(torch.bfloat16))  # torch: binary64 -> bfloat16


def brute_force(x, r, w, eps, code):
    """binary64 evaluation with numpy's reductions; the residual is rounded to
    the 16-bit type first (the op stores it), everything after is binary64."""
    f = (lambda a: a.view(np.float16).astype(np.float64)) if code == HF else \
        (lambda a: (a.astype(np.uint32) << 16).view(np.float32).astype(np.float64))
    s16 = to_16(f(x) + f(r), code)
    s = f(s16)
    rms = np.sqrt(np.mean(s * s, axis=-1, keepdims=True) + eps)
    return to_16(s / rms * f(w)[None, :], code), s16


# ---- the pins, each returning a failure message or None ----------------------------------
def pin_golden(golden, mutation=0):
    for name, c in golden.items():
        if c["kind"] != "fused":
            continue
        code = BF if c["dtype"] == "bf16" else HF
        out, res = oracle.fused_add_rmsnorm(c["x"], c["w"], c["r"], c["eps"], code, mutation=mutation)
        dr = oracle.ulp_distance(res, c["res"], code)
        if dr.max() != 0:
            return f"{name}: residual differs"
        d = oracle.ulp_distance(out, c["out"], code)
        if d.max() > 1:
            return f"{name}: output {d.max()} ulp"
        if (d != 0).mean() > 1e-3:
            return f"{name}: {(d != 0).mean():.1e} of outputs off by one ulp"
    return None


LIVE = [(64, 4096, BF, 1e-6, "bench"), (48, 5120, HF, 1e-6, "bench"), (16, 1000, BF, 2 ** -7, "reference_test"),
        (8, 32768, BF, 1e-6, "bench"), (32, 768, HF, 2 ** -7, "reference_test"), (200, 64, BF, 1e-5, "bench")]


def pin_torch_live(mutation=0):
    for i, (rows, hidden, code, eps, dist) in enumerate(LIVE):
        x, r, w = seeded(rows, hidden, code, 50 + i, dist)
        want_out, want_res = torch_formula(x, r, w, eps, code)
        out, res = oracle.fused_add_rmsnorm(x, w, r, eps, code, mutation=mutation)
        if not np.array_equal(res, want_res):
            return f"live {rows}x{hidden}: residual differs"
        d = oracle.ulp_distance(out, want_out, code)
        if d.max() > 1 or (d != 0).mean() > 1e-3:
            return f"live {rows}x{hidden}: output max {d.max()} ulp, {(d != 0).mean():.1e} off"
    return None


def pin_brute_force(mutation=0):
    for i, (rows, hidden, code) in enumerate([(16, 96, BF), (16, 130, HF), (4, 2048, BF), (9, 7, HF)]):
        x, r, w = seeded(rows, hidden, code, 90 + i)
        want_out, want_res = brute_force(x, r, w, 1e-6, code)
        out, res = oracle.fused_add_rmsnorm(x, w, r, 1e-6, code, mutation=mutation)
        if not np.array_equal(res, want_res):
            return f"brute {rows}x{hidden}: residual differs"
        if oracle.ulp_distance(out, want_out, code).max() > 1:
            return f"brute {rows}x{hidden}: output beyond 1 ulp of binary64"
    return None


def pin_closed_forms(mutation=0):
    for code in (BF, HF):
        rows, hidden = 6, 256
        _, _, w = seeded(1, hidden, code, 7)
        # constant rows c = +-2^k (x = c, r = 0) with eps = 0: out = sign(c) * w exactly
        cs = np.array([2.0 ** (k - 3) * (-1) ** k for k in range(rows)])
        x = to_16(np.repeat(cs[:, None], hidden, axis=1), code)
        r = np.zeros_like(x)
        out, res = oracle.fused_add_rmsnorm(x, w, r, 0.0, code, mutation=mutation)
        if not np.array_equal(res, x):
            return "constant rows: residual != x + 0"
        want = np.where(cs[:, None] < 0, w[None, :] ^ 0x8000, w[None, :]).astype(np.uint16)
        if not np.array_equal(out, want):
            return "constant rows: output != +-w"
        # power-of-two scaling of a row leaves the output unchanged (eps = 0)
        x, r, w2 = seeded(4, 512, code, 8)
        base, _ = oracle.fused_add_rmsnorm(x, w2, r, 0.0, code, mutation=mutation)
        f = oracle.to_f32(x, code).astype(np.float64) * 4.0
        g = oracle.to_f32(r, code).astype(np.float64) * 4.0
        scaled, _ = oracle.fused_add_rmsnorm(to_16(f, code), w2, to_16(g, code), 0.0, code, mutation=mutation)
        if not np.array_equal(base, scaled):
            return "scaling a row by 4 changed the output"
    return None


def pin_special_values(mutation=0):
    """The live torch formula on rows of special values (helpers.SPECIAL_PATTERNS:
    NaN, infinities, zero rows, binary32 overflow of a square and of the sum of
    squares, subnormals), also with a weight of special values
    (helpers.special_weight), with eps = 0 and 1e-6 and with eps that swamps the
    mean square or overflows binary32 (1, 1e30, 1e39, inf: the output goes to
    zero, NaN where a factor is infinite): the residual bit-exact and the output
    within 1 ulp, NaN where torch's is NaN (NaN bit patterns are not compared:
    torch's own differ between its vectorised and scalar paths)."""
    for code in (BF, HF):
        for hidden, weight in ((300, "plain"), (1024, "plain"), (520, "special")):
            x, r, w = special_inputs(28, hidden, TDT[code], hidden)
            if weight == "special":
                w = special_weight(w)
            x, r, w = tbits(x), tbits(r), tbits(w)
            for eps in (0.0, 1e-6, 1.0, 1e30, 1e39, float("inf")):
                want_out, want_res = torch_formula(x, r, w, eps, code)
                out, res = oracle.fused_add_rmsnorm(x, w, r, eps, code, mutation=mutation)
                if oracle.ulp_distance(res, want_res, code).max() != 0:
                    return f"special {hidden} eps {eps}: residual differs"
                d = oracle.ulp_distance(out, want_out, code)
                if d.max() > 1:
                    bad = SPECIAL_PATTERNS[int(np.argmax(d.max(axis=1))) % len(SPECIAL_PATTERNS)]
                    return f"special {hidden} eps {eps} {weight} weight: output {d.max()} ulp in a {bad!r} row"
    return None


def all_pins(golden, mutation=0):
    return [m for m in (pin_golden(golden, mutation), pin_torch_live(mutation), pin_brute_force(mutation),
                        pin_closed_forms(mutation), pin_special_values(mutation)) if m]


# ---- tests ---------------------------------------------------------------------------------
def test_oracle_matches_golden_vectors(golden):
    assert pin_golden(golden) is None


def test_oracle_matches_live_torch_formula():
    assert pin_torch_live() is None


def test_oracle_matches_binary64_brute_force():
    assert pin_brute_force() is None


def test_oracle_closed_forms():
    assert pin_closed_forms() is None


def test_oracle_special_values_match_torch():
    assert pin_special_values() is None


def test_binary64_squares_are_caught_only_by_binary32_overflow_rows(golden):
    """Summing the squares in binary64 (no binary32 overflow) agrees with the
    pins on ordinary rows; only rows whose binary32 sum of squares overflows
    (the special-value rows and the golden case made from them) tell it from
    the reference's formula."""
    m = oracle.MUTATIONS["binary64_squares"]
    assert pin_special_values(m) is not None
    assert "binary32_overflow" in (pin_golden(golden, m) or "")
    assert pin_torch_live(m) is None and pin_brute_force(m) is None and pin_closed_forms(m) is None


@pytest.mark.parametrize("name", sorted(oracle.MUTATIONS))
def test_planted_mistake_is_rejected(golden, name):
    failures = all_pins(golden, oracle.MUTATIONS[name])
    assert failures, f"no pin rejects the planted mistake {name!r}"


def test_streamer_golden(golden):
    for name, c in golden.items():
        if c["kind"] != "stream":
            continue
        code = BF if c["dtype"] == "bf16" else HF
        assert np.array_equal(oracle.streamer(c["x"], code, oracle.COPY), c["copy"]), name
        got = oracle.streamer(c["x"], code, oracle.RELU)
        # torch's bf16 relu canonicalises NaN payloads; compare NaN-ness there
        assert oracle.ulp_distance(got, c["relu"], code).max() == 0, name


def test_streamer_relu_matches_torch_cpu():
    for code in (BF, HF):
        allbits = np.arange(65536, dtype=np.uint32).astype(np.uint16).reshape(64, 1024)
        got = oracle.streamer(allbits, code, oracle.RELU)
        want = tbits(torch.relu(tfrom(allbits, code)))
        assert oracle.ulp_distance(got, want, code).max() == 0
        nonnan = (allbits & 0x7FFF) <= (0x7F80 if code == BF else 0x7C00)
        assert np.array_equal(got[nonnan], want[nonnan])   # incl. -0 kept as -0


def test_fp16_conversion_exhaustive_and_random():
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = oracle.to_f32(allh, HF)
    want = allh.view(np.float16).astype(np.float32)
    same = (f.view(np.uint32) == want.view(np.uint32)) | (np.isnan(f) & np.isnan(want))
    assert same.all()
    rng = np.random.default_rng(0)
    u = rng.integers(0, 2 ** 32, size=4_000_000, dtype=np.uint64).astype(np.uint32)
    edges = np.array([0x477FEFFF, 0x477FF000, 0x477FF001, 0x33000000, 0x33000001, 0x33800000, 0x387FE000,
                      0x387FF000, 0x38800000, 0x7F800000, 0xFF800000, 0x7FC00000, 0x00000001, 0x80000000],
                     dtype=np.uint32)
    vals = np.concatenate([u, edges]).view(np.float32)
    got = oracle.from_f32(vals, HF)
    with np.errstate(over="ignore"):   # values beyond binary16's range become inf, as intended
        want = vals.astype(np.float16).view(np.uint16)
    nan = np.isnan(vals)
    assert np.array_equal(got[~nan], want[~nan])
    assert ((got[nan] & 0x7FFF) > 0x7C00).all()


def test_bf16_conversion_random():
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    assert np.array_equal(oracle.to_f32(allh, BF).view(np.uint32), allh.astype(np.uint32) << 16)
    rng = np.random.default_rng(1)
    u = rng.integers(0, 2 ** 32, size=4_000_000, dtype=np.uint64).astype(np.uint32)
    ties = (rng.integers(0, 2 ** 16, size=100_000, dtype=np.uint64).astype(np.uint32) << 16) | 0x8000
    vals = np.concatenate([u, ties, np.array([0x7F7FFFFF, 0x7F7F8000, 0xFF7F8000], np.uint32)]).view(np.float32)
    got = oracle.from_f32(vals, BF)
    want = tbits(torch.from_numpy(vals.copy()).to(torch.bfloat16))
    nan = np.isnan(vals)
    assert np.array_equal(got[~nan], want[~nan])
    assert ((got[nan] & 0x7FFF) > 0x7F80).all()


def test_oracle_rmsnorm_plain_matches_torch():
    for code in (BF, HF):
        x, _, w = seeded(32, 1536, code, 3)
        want = tbits(torch.rms_norm(tfrom(x, code), (1536,), weight=tfrom(w, code), eps=1e-6))
        d = oracle.ulp_distance(oracle.rmsnorm(x, w, 1e-6, code), want, code)
        assert d.max() <= 1 and (d != 0).mean() < 1e-3


def test_oracle_rmsnorm_plain_special_values_match_torch():
    for code in (BF, HF):
        x, r, w = (tbits(t) for t in special_inputs(28, 520, TDT[code], 5))
        s = tbits(tfrom(x, code) + tfrom(r, code))          # the special rows as one input
        for eps in (0.0, 1e-6, 1e30, float("inf")):
            want = tbits(torch.rms_norm(tfrom(s, code), (520,), weight=tfrom(w, code), eps=eps))
            assert oracle.ulp_distance(oracle.rmsnorm(s, w, eps, code), want, code).max() <= 1, (code, eps)


def test_oracle_strided_rows_and_threads():
    x, r, w = seeded(40, 1000, BF, 4)
    want_out, want_res = oracle.fused_add_rmsnorm(x, w, r, 1e-6, BF)
    bx = np.zeros((40, 1024), np.uint16)
    br = np.zeros((40, 1030), np.uint16)
    bx[:, :1000] = x
    br[:, 3:1003] = r
    oracle.fused_add_rmsnorm_(bx[:, :1000], w, br[:, 3:1003], 1e-6, BF, threads=4)
    assert np.array_equal(bx[:, :1000], want_out) and np.array_equal(br[:, 3:1003], want_res)
    assert not bx[:, 1000:].any() and not br[:, :3].any() and not br[:, 1003:].any()


def test_oracle_rejects_bad_arguments():
    x = np.zeros((2, 8), np.uint16)
    with pytest.raises(ValueError):
        oracle.fused_add_rmsnorm(x, np.zeros(8, np.uint16), x, 1e-6, 7)


# ---- FP8 (e4m3fn) output --------------------------------------------------------------------
def torch_quantise(y_bits, code):
    """Per-row dynamic quantisation of a 16-bit output as torch evaluates it."""
    y = tfrom(y_bits, code).float()
    scale = torch.clamp(y.abs().amax(-1, keepdim=True) / 448.0, min=torch.finfo(torch.float32).tiny)
    q = (y * (1.0 / scale)).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q.view(torch.uint8).numpy(), scale.reshape(-1).numpy()


def test_e4m3_conversion_matches_torch():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    pts = np.unique(codes[np.isfinite(codes)])
    mids = ((pts[:-1].astype(np.float64) + pts[1:]) / 2).astype(np.float32)
    u = np.concatenate([pts.astype(np.float32), mids]).view(np.uint32).astype(np.int64)
    near = np.concatenate([u + k for k in range(-3, 4)])
    near = near[(near >= 0) & (near < 2 ** 32)].astype(np.uint32).view(np.float32)
    rng = np.random.default_rng(2)
    vals = np.concatenate([near, rng.uniform(-600, 600, 2_000_000).astype(np.float32),
                           (rng.standard_normal(1_000_000) * 1e-2).astype(np.float32),
                           np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 464.0, 480.0], np.float32)])
    got = oracle.e4m3_from_f32(vals)
    want = torch.from_numpy(vals).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got, want)


def test_oracle_fp8_quantisation_stage_matches_torch():
    """The oracle's q and scale equal torch's quantisation of the oracle's own
    16-bit output (so the FP8 stage is pinned independently of y)."""
    cases = [(64, 4096, BF, "bench"), (32, 5120, HF, "bench"), (16, 1000, BF, "reference_test"), (8, 13, HF, "bench")]
    for i, (rows, hidden, code, dist) in enumerate(cases):
        x, r, w = seeded(rows, hidden, code, 300 + i, dist)
        x[0, :] = 0
        r[0, :] = 0                                  # zero row
        y, res = oracle.fused_add_rmsnorm(x, w, r, 1e-6, code)
        q, sc, res8 = oracle.fused_add_rmsnorm_fp8(x, w, r, 1e-6, code)
        assert np.array_equal(res8, res)
        tq, tsc = torch_quantise(y, code)
        assert np.array_equal(sc, tsc)
        assert oracle.e4m3_ulp_distance(q, tq).max() == 0


def torch_quantise_ub(y, code, scale_ub):
    """torch's per-row quantisation of 16-bit outputs y with the row maximum
    bounded above (binary32 on the CPU): amax' = amax where not amax >
    scale_ub, else scale_ub (torch.where keeps a NaN maximum, and a NaN bound
    bounds nothing), scale = clamp(amax' / 448, min=FLT_MIN)."""
    yf = tfrom(y, code).float()
    amax = yf.abs().amax(-1, keepdim=True)
    ub = torch.tensor(scale_ub, dtype=torch.float32)
    amax = torch.where(amax > ub, ub, amax)
    sc = torch.clamp(amax / 448.0, min=torch.finfo(torch.float32).tiny)
    q = (yf * (1.0 / sc)).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q.view(torch.uint8).numpy(), sc.view(-1).numpy()


UB_BOUNDS = [0.5, 2.0, 3.5, 1e-30, 1e30, float("inf"), 0.0, float("nan")]


def test_oracle_fp8_ub_matches_torch_and_the_unbounded_form():
    """The bounded form: q and the scales equal torch's bounded quantisation of
    the oracle's own 16-bit output bit for bit (NaN where torch's is), on
    ordinary and special rows and bounds that bound most rows, some, none
    (huge, infinite, NaN) and all down to the FLT_MIN floor (tiny, zero); with
    a bound no row reaches, they equal the unbounded C oracle's bit for bit;
    and every bounded row's scale is exactly max(bound / 448, FLT_MIN)."""
    tiny = np.float32(np.finfo(np.float32).tiny)
    for code in (BF, HF):
        for i, (rows, hidden, kind) in enumerate([(64, 4096, "bench"), (16, 1000, "reference_test"),
                                                  (28, 520, "special")]):
            if kind == "special":
                x, r, w = (tbits(t) for t in special_inputs(rows, hidden, TDT[code], 31 + i))
            else:
                x, r, w = seeded(rows, hidden, code, 700 + i, kind)
            y, res = oracle.fused_add_rmsnorm(x, w, r, 1e-6, code)
            q0, sc0, _ = oracle.fused_add_rmsnorm_fp8(x, w, r, 1e-6, code)
            amax = np.abs(oracle.to_f32(y, code)).max(axis=1)
            for ub in UB_BOUNDS:
                q, sc, res8 = oracle.fused_add_rmsnorm_fp8_ub(x, w, r, 1e-6, code, ub)
                assert np.array_equal(res8, res), (code, kind, ub)
                tq, tsc = torch_quantise_ub(y, code, ub)
                assert np.array_equal(sc.view(np.uint32), tsc.view(np.uint32)) or \
                    np.array_equal(sc, tsc, equal_nan=True), (code, kind, ub)
                assert oracle.e4m3_ulp_distance(q, tq).max() == 0, (code, kind, ub)
                with np.errstate(invalid="ignore"):
                    bounded = amax > np.float32(ub)
                    free = ~bounded
                want = max(np.float32(np.float32(ub) / np.float32(448.0)), tiny)
                assert (sc[bounded] == want).all(), (code, kind, ub)
                assert np.array_equal(sc[free], sc0[free], equal_nan=True), (code, kind, ub)
                if free.any():
                    assert oracle.e4m3_ulp_distance(q[free], q0[free]).max() == 0, (code, kind, ub)
                if ub in (1e30, float("inf"), float("nan")):
                    assert not bounded.any()


def test_planted_fp8_ub_mistake_is_rejected():
    """Bounding the scale by the bound instead of the row maximum (scale =
    min(amax / 448, bound)), planted in the oracle, fails the torch pin."""
    x, r, w = seeded(64, 4096, BF, 700, "bench")
    y, _ = oracle.fused_add_rmsnorm(x, w, r, 1e-6, BF)
    for ub in (0.5, 2.0, 3.5):
        q, sc, _ = oracle.fused_add_rmsnorm_fp8_ub(x, w, r, 1e-6, BF, ub, bound_scale=True)
        tq, tsc = torch_quantise_ub(y, BF, ub)
        assert not np.array_equal(sc, tsc) or oracle.e4m3_ulp_distance(q, tq).max() > 0, ub


STATIC_SCALES = [0.01, 1.0, 3.0, 7e-4, 2.0 ** -140, 1e30, 0.0, float("inf"), float("nan")]


def torch_quantise_static(y, code, scale):
    """torch's static per-tensor quantisation of 16-bit outputs y:
    e4m3fn(clamp(y * reciprocal(scale), -448, 448)) in binary32 on the CPU."""
    yf = tfrom(y, code).float()
    q = (yf * torch.reciprocal(torch.tensor(scale, dtype=torch.float32))).clamp(-448.0, 448.0)
    return q.to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_oracle_fp8_static_quantisation_matches_torch():
    """The static form: the residual is the fused oracle's, and q equals torch's
    quantisation of the oracle's own 16-bit output with the given scale, bit for
    bit (NaN where torch's is NaN), on ordinary and special rows and for scales
    that are ordinary, subnormal, huge, zero, infinite and NaN."""
    for code in (BF, HF):
        for i, (rows, hidden, kind) in enumerate([(64, 4096, "bench"), (16, 1000, "reference_test"),
                                                  (28, 520, "special")]):
            if kind == "special":
                x, r, w = (tbits(t) for t in special_inputs(rows, hidden, TDT[code], 11 + i))
            else:
                x, r, w = seeded(rows, hidden, code, 500 + i, kind)
            y, res = oracle.fused_add_rmsnorm(x, w, r, 1e-6, code)
            for scale in STATIC_SCALES:
                q, res8 = oracle.fused_add_rmsnorm_fp8_static(x, w, r, 1e-6, code, scale)
                assert np.array_equal(res8, res), (code, kind, scale)
                d = oracle.e4m3_ulp_distance(q, torch_quantise_static(y, code, scale))
                assert d.max() == 0, (code, kind, scale)


def test_oracle_fp8_static_and_group_match_golden(golden):
    """The torch-made golden vectors of the static and per-group FP8 forms: the
    residual bit-exact; where the oracle's 16-bit output equals torch's (every
    element for the static form, every element of a group for the per-group
    form) q and the scales equal torch's bit for bit, and everywhere q is the
    quantisation of a y within one 16-bit ulp of torch's output."""
    from helpers import assert_fp8_from_y_within_one_ulp, assert_group_scales
    seen = set()
    for name, c in golden.items():
        if c["kind"] not in ("fp8_static", "fp8_group"):
            continue
        seen.add(c["kind"])
        code = BF if c["dtype"] == "bf16" else HF
        dt = TDT[code]
        y, _ = oracle.fused_add_rmsnorm(c["x"], c["w"], c["r"], c["eps"], code)
        same = oracle.ulp_distance(y, c["out"], code) == 0
        if c["kind"] == "fp8_static":
            q, res = oracle.fused_add_rmsnorm_fp8_static(c["x"], c["w"], c["r"], c["eps"], code, c["scale"])
            isc = np.float32(1.0) / np.float32(c["scale"])
            assert np.array_equal(q[same], c["q"][same]), name
        else:
            q, sc, res = oracle.fused_add_rmsnorm_fp8_group(c["x"], c["w"], c["r"], c["eps"], code)
            gsame = same.reshape(same.shape[0], -1, 128).all(-1)
            assert np.array_equal(sc[gsame], c["scale"][gsame], equal_nan=True), name
            assert_group_scales(sc, c["out"], 128, dt, name)
            with np.errstate(divide="ignore"):
                isc = np.repeat(np.float32(1.0) / sc, 128, axis=1)
            eq = oracle.e4m3_ulp_distance(q, c["q"]) == 0
            assert eq[np.repeat(gsame, 128, axis=1)].all(), name
        assert oracle.ulp_distance(res, c["res"], code).max() == 0, name
        assert_fp8_from_y_within_one_ulp(q, c["out"], isc, dt, name)
    assert seen == {"fp8_static", "fp8_group"}


def test_planted_fp8_static_mistakes_are_rejected():
    """Two plausible mistakes in the static step, planted in a copy of the
    oracle's composition, each fail the torch pin above: the reciprocal of the
    scale rounded to the tensor's 16-bit type, and the clamp to +-448 left out
    (the e4m3fn cast then gives NaN past 464)."""
    x, r, w = seeded(64, 4096, BF, 500, "bench")
    y, _ = oracle.fused_add_rmsnorm(x, w, r, 1e-6, BF)
    yf = oracle.to_f32(y, BF)
    for scale in (3.0, 7e-4):
        want = torch_quantise_static(y, BF, scale)
        isc = np.float32(1.0) / np.float32(scale)
        isc16 = oracle.to_f32(oracle.from_f32(np.array([isc], np.float32), BF), BF)[0]
        rounded = oracle.e4m3_from_f32(np.clip(yf * isc16, -448, 448).astype(np.float32))
        unclamped = oracle.e4m3_from_f32((yf * isc).astype(np.float32))
        assert oracle.e4m3_ulp_distance(rounded, want).max() > 0, scale
        if scale == 7e-4:    # outputs past 448 only with the small scale
            assert oracle.e4m3_ulp_distance(unclamped, want).max() > 0


def torch_quantise_group(y, code, group=128):
    """torch's per-token-group quantisation of 16-bit outputs y (binary32 on
    the CPU): per `group` elements, scale = clamp(amax / 448, min=FLT_MIN),
    q = e4m3fn(clamp(y * (1 / scale), -448, 448))."""
    yf = tfrom(y, code).float()
    rows, hidden = yf.shape
    g = yf.view(rows, hidden // group, group)
    sc = torch.clamp(g.abs().amax(-1, keepdim=True) / 448.0, min=torch.finfo(torch.float32).tiny)
    q = (g * (1.0 / sc)).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q.view(rows, hidden).view(torch.uint8).numpy(), sc.view(rows, -1).numpy()


def test_oracle_fp8_group_matches_torch():
    """The FP8 output with a scale per 128 elements: the residual is the fused
    oracle's, and q and the scales equal torch's per-group quantisation of the
    oracle's own 16-bit output bit for bit (NaN where torch's is NaN), on
    ordinary rows, rows with an outlier and rows of special values."""
    for code in (BF, HF):
        for i, (rows, hidden, kind) in enumerate([(64, 4096, "bench"), (32, 1024, "outliers"), (28, 640, "special")]):
            if kind == "special":
                x, r, w = (tbits(t) for t in special_inputs(rows, hidden, TDT[code], 21 + i))
            else:
                x, r, w = seeded(rows, hidden, code, 600 + i, kind)
            y, res = oracle.fused_add_rmsnorm(x, w, r, 1e-6, code)
            q, sc, resg = oracle.fused_add_rmsnorm_fp8_group(x, w, r, 1e-6, code)
            assert np.array_equal(resg, res), (code, kind)
            tq, tsc = torch_quantise_group(y, code)
            assert np.array_equal(sc.view(np.uint32), tsc.view(np.uint32)) or \
                np.array_equal(sc, tsc, equal_nan=True), (code, kind)
            assert oracle.e4m3_ulp_distance(q, tq).max() == 0, (code, kind)


def test_planted_fp8_group_mistakes_are_rejected():
    """Groups of 32 (an MX block) instead of 128, and the FLT_MIN floor of the
    scale left out (a zero group then gives NaN codes), each fail the torch pin
    above on rows that include zero rows."""
    x, r, w = (tbits(t) for t in special_inputs(28, 640, torch.bfloat16, 21))
    y, _ = oracle.fused_add_rmsnorm(x, w, r, 1e-6, BF)
    tq, tsc = torch_quantise_group(y, BF)
    q32, sc32, _ = oracle.fused_add_rmsnorm_fp8_group(x, w, r, 1e-6, BF, group=32)
    assert oracle.e4m3_ulp_distance(q32, tq).max() > 0
    qnf, scnf, _ = oracle.fused_add_rmsnorm_fp8_group(x, w, r, 1e-6, BF, floor=False)
    assert oracle.e4m3_ulp_distance(qnf, tq).max() > 0 or not np.array_equal(scnf, tsc, equal_nan=True)


def test_oracle_fp8_matches_golden(golden):
    for name, c in golden.items():
        if c["kind"] != "fp8":
            continue
        code = BF if c["dtype"] == "bf16" else HF
        q, sc, res = oracle.fused_add_rmsnorm_fp8(c["x"], c["w"], c["r"], c["eps"], code)
        assert oracle.ulp_distance(res, c["res"], code).max() == 0, name
        y, _ = oracle.fused_add_rmsnorm(c["x"], c["w"], c["r"], c["eps"], code)
        same = np.all(oracle.ulp_distance(y, c["out"], code) == 0, axis=1)
        assert same.mean() >= 0.5, name
        d = oracle.e4m3_ulp_distance(q, c["q"])
        assert d[same].max(initial=0) == 0, name          # rows whose y matches: bit-exact
        assert np.array_equal(sc[same], c["scale"][same], equal_nan=True), name
        assert d.max() <= 1, name                          # elsewhere within one FP8 step


def test_planted_fp8_mistake_is_rejected():
    """Quantising with a scale of amax / 240 (the e4m3fnuz maximum) instead of
    448 fails the torch pin of the quantisation stage."""
    x, r, w = seeded(16, 512, BF, 9)
    y, _ = oracle.fused_add_rmsnorm(x, w, r, 1e-6, BF)
    tq, tsc = torch_quantise(y, BF)
    yf = oracle.to_f32(y, BF)
    bad_scale = np.maximum(np.abs(yf).max(-1) / np.float32(240.0), np.finfo(np.float32).tiny).astype(np.float32)
    bad_q = oracle.e4m3_from_f32(np.clip(yf * (np.float32(1.0) / bad_scale)[:, None], -448, 448))
    assert not np.array_equal(bad_scale, tsc) and oracle.e4m3_ulp_distance(bad_q, tq).max() > 0


# ---- the partial-sum form (reduce + residual-add + RMSNorm) ---------------------------------
def torch_reduce_formula(parts, r, w, eps, code):
    """The all-reduce of the parts as torch evaluates it (binary32 adds in part
    order, one conversion to the 16-bit type), followed by the reference test's
    formula (test/test_hp_rms_norm.py:6-19)."""
    acc = tfrom(parts[0], code).float()
    for p in parts[1:]:
        acc = acc + tfrom(p, code).float()
    return torch_formula(tbits(acc.to(TDT[code])), r, w, eps, code)


def pin_reduce_torch_live(mutation=0):
    for code in (BF, HF):
        for nparts in (1, 2, 3, 8):
            parts = [seeded(16, 384, code, 200 + g)[0] for g in range(nparts)]
            _, r, w = seeded(16, 384, code, 199)
            out, res = oracle.reduce_add_rmsnorm(parts, w, r, 1e-6, code, mutation=mutation)
            want_out, want_res = torch_reduce_formula(parts, r, w, 1e-6, code)
            if oracle.ulp_distance(res, want_res, code).max() != 0:
                return f"P={nparts}: residual differs from torch"
            if oracle.ulp_distance(out, want_out, code).max() > 1:
                return f"P={nparts}: output beyond 1 ulp of torch"
    return None


def bits16(values, code):
    return tbits(torch.tensor(values, dtype=torch.float64).to(TDT[code]))


def pin_reduce_closed_forms(mutation=0):
    """Residual values fixed by the definition, with u = ulp(1) of the type:
    1 + u/2 + u/2 = 1 + u when rounded once (rounding after each addition ties
    to 1 twice); (1 + u/2) rounds to 1 before the residual u/2 is added, so the
    sum is 1, not 1 + u; 2^24 + 1 - 2^24 = 0 in binary32 left to right (the
    reversed order gives 1)."""
    for code, u in ((BF, 2.0 ** -7), (HF, 2.0 ** -10)):
        w = bits16([1.0] * 8, code)

        def res_of(part_values, r_value):
            parts = [bits16([[v] * 8], code) for v in part_values]
            _, res = oracle.reduce_add_rmsnorm(parts, w, bits16([[r_value] * 8], code), 1e-6, code,
                                               mutation=mutation)
            return oracle.to_f32(res, code)[0]
        if not np.all(res_of([1.0, u / 2, u / 2], 0.0) == np.float32(1 + u)):
            return "1 + u/2 + u/2 is not rounded once"
        if not np.all(res_of([1.0, u / 2], u / 2) == np.float32(1.0)):
            return "the reduced sum is not rounded before the residual add"
        # 2^24 is a bfloat16 value but not a binary16 one (max 65504)
        if code == BF and not np.all(res_of([2.0 ** 24, 1.0, -2.0 ** 24], 0.0) == 0.0):
            return "parts are not summed left to right"
    return None


def test_reduce_oracle_matches_live_torch_formula():
    assert pin_reduce_torch_live() is None


def test_reduce_oracle_closed_forms():
    assert pin_reduce_closed_forms() is None


def test_reduce_oracle_with_one_part_is_the_fused_op():
    x, r, w = seeded(32, 520, BF, 3)
    out, res = oracle.reduce_add_rmsnorm([x], w, r, 1e-6, BF)
    want_out, want_res = oracle.fused_add_rmsnorm(x, w, r, 1e-6, BF)
    assert np.array_equal(out, want_out) and np.array_equal(res, want_res)


@pytest.mark.parametrize("name", sorted(oracle.REDUCE_MUTATIONS))
def test_planted_reduce_mistake_is_rejected(name):
    m = oracle.REDUCE_MUTATIONS[name]
    failures = [f for f in (pin_reduce_torch_live(m), pin_reduce_closed_forms(m)) if f]
    assert failures, f"no pin rejects the planted mistake {name!r}"
