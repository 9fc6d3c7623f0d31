"""Writes tests/golden/golden.npz + golden.json: seeded input/output vectors of
the reference's own test oracle, evaluated with torch on the CPU.

The formula is the reference's test oracle (test/test_hp_rms_norm.py:6-19):
    inp_res = inp + res
    out = torch.rms_norm(inp_res, normalized_shape=(H,), weight=weight, eps=eps)
and the streamer's pinned behaviour (test/test_relu.py:24: out == inp), plus
torch.relu for the true-ReLU variant.  The reference package itself is not
imported (it needs its CUDA extension); only torch runs here.

Run from the repository root:  python tests/golden/make_golden.py
"""
import json
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def fused_case(name, rows, hidden, dtype, eps, dist, seed, special=None):
    g = torch.Generator().manual_seed(seed)
    if dist == "reference_test":          # test/test_hp_rms_norm.py:29-31: all N(0, 0.1)
        x = torch.normal(0, 0.1, (rows, hidden), generator=g)
        r = torch.normal(0, 0.1, (rows, hidden), generator=g)
        w = torch.normal(0, 0.1, (hidden,), generator=g)
    else:                                  # the benchmark distribution: N(0,1), N(0,1), N(1, 0.1)
        x = torch.randn((rows, hidden), generator=g)
        r = torch.randn((rows, hidden), generator=g)
        w = 1 + 0.1 * torch.randn((hidden,), generator=g)
        if dist == "outliers":             # 1% of input entries scaled by 50
            m = torch.rand((rows, hidden), generator=g) < 0.01
            x = torch.where(m, x * 50, x)
    x, r, w = x.to(dtype), r.to(dtype), w.to(dtype)
    if special is not None:
        special(x, r, w)
    inp_res = x + r
    out = torch.rms_norm(inp_res, normalized_shape=(hidden,), weight=w, eps=eps)
    return name, {"kind": "fused", "dtype": "bf16" if dtype == torch.bfloat16 else "fp16",
                  "eps": eps, "rows": rows, "hidden": hidden}, \
        {"x": bits(x), "r": bits(r), "w": bits(w), "out": bits(out), "res": bits(inp_res)}


def sp_zero_and_huge(x, r, w):
    x[0].zero_(); r[0].zero_()             # all-zero row: out = 0
    x[1].fill_(1e30); r[1].fill_(1e30)     # squares overflow fp32: inv = 0
    x[2, 5] = float("nan")                 # NaN poisons one row's output


def sp_fp16_overflow(x, r, w):
    x[0, :4] = 60000.0; r[0, :4] = 60000.0   # sum rounds to inf
    x[1].fill_(2.0 ** -20); r[1].fill_(2.0 ** -20)  # subnormal sums


def sp_binary32_overflow(x, r, w):
    """Rows whose binary32 sum of squares overflows while their mean would
    not (torch's fp32 sum makes the inverse 0, a binary64 sum would not),
    and rows of subnormals, with eps = 0."""
    r.zero_()
    x[0].fill_(3e18)                       # every square finite, the sum infinite
    x[1, 7] = 1e20                         # one square infinite
    x[2].fill_(1e-20)                      # squares that are binary32 subnormals
    x[3, :256] = 1e-39                     # half the row bf16 subnormals
    x[4].zero_()                           # zero row, eps = 0: 0 * inf = NaN


def sp_constant_rows(x, r, w):
    x.zero_(); r.zero_()
    for i in range(x.shape[0]):
        x[i].fill_(2.0 ** (i - 3) * (-1) ** i)


def fp8_case(name, rows, hidden, dtype, eps, seed, special=None):
    """The fused op's output quantised per row to float8_e4m3fn, as torch
    evaluates it: scale = max(amax|y| / 448, FLT_MIN); q = e4m3fn(clamp(y *
    (1 / scale), -448, 448)).  Input x is not modified by the FP8 variant."""
    name, meta, arrs = fused_case(name, rows, hidden, dtype, eps, "bench", seed, special)
    y = torch.from_numpy(arrs["out"].view(np.int16)).view(dtype)
    yf = y.float()
    amax = yf.abs().amax(-1, keepdim=True)
    scale = torch.clamp(amax / 448.0, min=torch.finfo(torch.float32).tiny)
    q = (yf * (1.0 / scale)).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    meta["kind"] = "fp8"
    arrs["q"] = q.view(torch.uint8).numpy().copy()
    arrs["scale"] = scale.reshape(-1).numpy().copy()
    return name, meta, arrs


def fp8_static_case(name, rows, hidden, dtype, eps, seed, scale, special=None):
    """The fused op's output quantised with one given scale for every row, as
    torch evaluates it: q = e4m3fn(clamp(y * reciprocal(scale), -448, 448))."""
    name, meta, arrs = fused_case(name, rows, hidden, dtype, eps, "bench", seed, special)
    y = torch.from_numpy(arrs["out"].view(np.int16)).view(dtype).float()
    q = (y * torch.reciprocal(torch.tensor(scale, dtype=torch.float32))).clamp(-448.0, 448.0)
    meta["kind"] = "fp8_static"
    meta["scale"] = scale
    arrs["q"] = q.to(torch.float8_e4m3fn).view(torch.uint8).numpy().copy()
    return name, meta, arrs


def fp8_group_case(name, rows, hidden, dtype, eps, seed, special=None):
    """The fused op's output quantised with one scale per 128 consecutive
    elements, as torch evaluates it: per group scale = max(amax|y| / 448,
    FLT_MIN), q = e4m3fn(clamp(y * (1 / scale), -448, 448))."""
    name, meta, arrs = fused_case(name, rows, hidden, dtype, eps, "bench", seed, special)
    y = torch.from_numpy(arrs["out"].view(np.int16)).view(dtype).float().view(rows, hidden // 128, 128)
    scale = torch.clamp(y.abs().amax(-1, keepdim=True) / 448.0, min=torch.finfo(torch.float32).tiny)
    q = (y * (1.0 / scale)).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    meta["kind"] = "fp8_group"
    arrs["q"] = q.view(rows, hidden).view(torch.uint8).numpy().copy()
    arrs["scale"] = scale.view(rows, -1).numpy().copy()
    return name, meta, arrs


def sp_fp8_rows(x, r, w):
    x[0].zero_(); r[0].zero_()             # all-zero row: scale = FLT_MIN, q = 0
    x[1, 3] = float("nan")                 # NaN row: NaN scale, NaN outputs
    x[2] *= 1e-3; r[2] *= 1e-3             # small row: same q as a scaled row


def stream_case(name, rows, hidden, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((rows, hidden), generator=g).to(dtype)
    specials = [0.0, -0.0, float("nan"), float("inf"), -float("inf"), 1e-40, -1e-40, -1.0, 1.0]
    x[0, :len(specials)] = torch.tensor(specials).to(dtype)
    return name, {"kind": "stream", "dtype": "bf16" if dtype == torch.bfloat16 else "fp16",
                  "rows": rows, "hidden": hidden}, \
        {"x": bits(x), "copy": bits(x.clone()), "relu": bits(torch.relu(x))}


def main():
    bf, hf = torch.bfloat16, torch.float16
    cases = [
        fused_case("bf16_4x4096_bench", 4, 4096, bf, 1e-6, "bench", 1),
        fused_case("bf16_3x1024_reftest", 3, 1024, bf, 2.0 ** -7, "reference_test", 2),
        fused_case("bf16_5x128_reftest", 5, 128, bf, 2.0 ** -7, "reference_test", 3),
        fused_case("fp16_3x5120_bench", 3, 5120, hf, 1e-6, "bench", 4),
        fused_case("fp16_2x7168_bench", 2, 7168, hf, 1e-6, "bench", 5),
        fused_case("bf16_1x32768_bench", 1, 32768, bf, 1e-6, "bench", 6),
        fused_case("bf16_2x8192_outliers", 2, 8192, bf, 1e-6, "outliers", 7),
        fused_case("bf16_3x1000_tail", 3, 1000, bf, 1e-6, "bench", 8),
        fused_case("fp16_2x13_tail", 2, 13, hf, 1e-6, "bench", 9),
        fused_case("bf16_4x256_special", 4, 256, bf, 1e-6, "bench", 10, sp_zero_and_huge),
        fused_case("fp16_2x256_special", 2, 256, hf, 1e-6, "bench", 11, sp_fp16_overflow),
        fused_case("bf16_6x512_constant_eps0", 6, 512, bf, 0.0, "bench", 12, sp_constant_rows),
        fused_case("bf16_6x512_binary32_overflow_eps0", 6, 512, bf, 0.0, "bench", 18, sp_binary32_overflow),
        fp8_case("fp8_bf16_4x4096", 4, 4096, bf, 1e-6, 15),
        fp8_case("fp8_fp16_3x5120", 3, 5120, hf, 1e-6, 16),
        fp8_case("fp8_bf16_4x1000_tail", 4, 1000, bf, 1e-6, 17, sp_fp8_rows),
        fp8_static_case("fp8_static_bf16_4x4096", 4, 4096, bf, 1e-6, 19, 0.02),
        fp8_static_case("fp8_static_fp16_3x1000_tail", 3, 1000, hf, 1e-6, 20, 0.01, sp_fp8_rows),
        fp8_group_case("fp8_group_bf16_4x4096", 4, 4096, bf, 1e-6, 21),
        fp8_group_case("fp8_group_fp16_3x5120", 3, 5120, hf, 1e-6, 22),
        fp8_group_case("fp8_group_bf16_4x1024_special", 4, 1024, bf, 1e-6, 23, sp_fp8_rows),
        stream_case("stream_bf16_3x384", 3, 384, bf, 13),
        stream_case("stream_fp16_2x1000", 2, 1000, hf, 14),
    ]
    arrays, meta = {}, {"torch": torch.__version__, "cases": {}}
    for name, m, arrs in cases:
        meta["cases"][name] = m
        for k, v in arrs.items():
            arrays[f"{name}/{k}"] = v
    np.savez_compressed(os.path.join(HERE, "golden.npz"), **arrays)
    with open(os.path.join(HERE, "golden.json"), "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)
    print("wrote", len(cases), "cases")


if __name__ == "__main__":
    main()
