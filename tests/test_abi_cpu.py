"""The C ABI of libhprms.so, on the CPU: the library loads, exports every
function include/hp_rms_norm_amd.h declares, rejects bad arguments with a
status and a message before touching a device, and its dispatch table maps
every hidden size to a kernel that is built."""
import ctypes
import os
import re

import pytest

from hp_rms_norm_amd import abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hp_rms_norm_amd.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hprms_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_function():
    names = declared_functions()
    assert len(names) >= 7
    lib = abi.lib()
    for n in names:
        assert hasattr(lib, n), f"{n} declared in the header but not exported"
    assert set(names) == set(abi.SYMBOLS)


def test_abi_version_matches_header():
    m = re.search(r"#define HPRMS_ABI_VERSION (\d+)", open(HEADER).read())
    assert abi.lib().hprms_abi_version() == int(m.group(1))


def test_status_codes_match_header():
    text = open(HEADER).read()
    for name, val in (("HPRMS_E_INVALID", abi.HPRMS_E_INVALID), ("HPRMS_E_LAUNCH", abi.HPRMS_E_LAUNCH),
                      ("HPRMS_E_RANGE", abi.HPRMS_E_RANGE)):
        assert re.search(rf"#define {name} \({val}\)", text), name


def fused(**kw):
    a = dict(input=0x1000, weight=0x2000, residual=0x3000, rows=4, hidden=4096, si=4096, sr=4096,
             dtype=abi.DTYPE_BF16, eps=1e-6)
    a.update(kw)
    return abi.lib().hprms_fused_add_rmsnorm(a["input"], a["weight"], a["residual"], a["rows"], a["hidden"],
                                             a["si"], a["sr"], a["dtype"], a["eps"], None)


@pytest.mark.parametrize("kw,msg", [
    (dict(dtype=2), "dtype"),
    (dict(rows=-1), "rows"),
    (dict(hidden=0), "hidden"),
    (dict(si=100), "input row stride"),
    (dict(sr=100), "residual row stride"),
    (dict(eps=-1.0), "eps"),
    (dict(input=0), "null"),
    (dict(residual=0), "null"),
    (dict(weight=0), "null"),
    (dict(residual=0x1000), "alias"),
])
def test_fused_rejects_bad_arguments(kw, msg):
    assert fused(**kw) == abi.HPRMS_E_INVALID
    assert msg in abi.last_error()


def test_fused_rejects_hidden_beyond_maximum():
    assert fused(hidden=(1 << 24) + 8, si=(1 << 24) + 8, sr=(1 << 24) + 8) == abi.HPRMS_E_RANGE


def test_rows_spanning_more_than_2_pow_56_bytes_are_rejected():
    """No buffer spans 2^56 bytes; such a call is a range error before any
    launch (the kernels' 64-bit row offsets would overflow past it)."""
    L = abi.lib()
    big = 1 << 40                                          # elements between rows
    assert fused(rows=1 << 16, si=big) == abi.HPRMS_E_RANGE    # 2^16 rows x 2^41 bytes = 2^57
    assert "2^56" in abi.last_error()
    assert fused(rows=1 << 16, sr=big) == abi.HPRMS_E_RANGE
    assert fused(rows=2, si=(1 << 62) + 4096) == abi.HPRMS_E_RANGE       # the stride alone overflows
    assert fused(rows=0, si=big) == abi.HPRMS_OK                         # nothing to do
    assert L.hprms_streamer(0x1000, 0x2000, 1 << 16, 64, big, 64, 0, 0, None) == abi.HPRMS_E_RANGE
    assert L.hprms_rmsnorm(0x1000, 0x2000, 0x3000, 1 << 16, 64, big, 64, 0, 1e-6, None) == abi.HPRMS_E_RANGE


def test_batch_invariant_mode_picks_the_shape_by_width_alone():
    """With the mode on, every row count takes the configuration the table
    gives a large batch (latency, wide, one- and two-wave rows are row-count
    rules); with it off, few rows take the latency rows.  The mode is
    process-wide and restored here."""
    previous = abi.set_batch_invariant(False)
    try:
        assert not abi.batch_invariant()
        for hidden in (1024, 2048, 3072, 4096, 6144, 8192, 16384, 32768, 4097):
            default = {n: abi.select_config(n, hidden, abi.DTYPE_BF16, 0).as_tuple()[:5] for n in (1, 1500, 1 << 20)}
            assert abi.set_batch_invariant(True) is False
            inv = {n: abi.select_config(n, hidden, abi.DTYPE_BF16, 0).as_tuple()[:5]
                   for n in (1, 8, 300, 1024, 1500, 2048, 3000, 4096, 1 << 20)}
            assert abi.set_batch_invariant(False) is True
            assert len(set(inv.values())) == 1, (hidden, inv)
            assert inv[1 << 20] == default[1 << 20]
        assert abi.select_config(8, 4096, abi.DTYPE_BF16, 0).as_tuple() != \
            abi.select_config(1 << 20, 4096, abi.DTYPE_BF16, 0).as_tuple()
        assert abi.lib().hprms_set_batch_invariant(2) == abi.HPRMS_E_INVALID
    finally:
        abi.set_batch_invariant(previous)


def test_batch_invariant_mode_from_the_environment():
    import subprocess
    import sys
    code = ("import sys; sys.path.insert(0, %r); from hp_rms_norm_amd import abi; "
            "print(abi.batch_invariant())") % ROOT
    for env_value, want in (("1", "True"), ("0", "False"), ("", "False")):
        env = dict(os.environ, HPRMS_BATCH_INVARIANT=env_value)
        out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, check=True)
        assert out.stdout.strip() == want, (env_value, out.stdout, out.stderr)


def test_zero_rows_is_a_no_op_without_pointers():
    assert fused(rows=0, input=0, weight=0, residual=0) == abi.HPRMS_OK


def test_streamer_and_plain_reject_bad_arguments():
    L = abi.lib()
    assert L.hprms_streamer(0x1000, 0x2000, 4, 64, 64, 64, 0, 5, None) == abi.HPRMS_E_INVALID
    assert "op" in abi.last_error()
    assert L.hprms_streamer(0x1000, 0x2000, 4, 64, 32, 64, 0, 0, None) == abi.HPRMS_E_INVALID
    assert L.hprms_streamer(0, 0, 0, 64, 64, 64, 0, 0, None) == abi.HPRMS_OK
    # a row's buffer resource spans 2 * hidden bytes, below 2^31
    assert L.hprms_streamer(0, 0, 0, 1 << 30, 1 << 30, 1 << 30, 0, 0, None) == abi.HPRMS_E_RANGE
    assert "2^30" in abi.last_error()
    assert L.hprms_streamer(0, 0, 0, (1 << 30) - 1, 1 << 30, 1 << 30, 0, 0, None) == abi.HPRMS_OK
    assert L.hprms_rmsnorm(0x1000, 0x2000, 0, 4, 64, 64, 64, 0, 1e-6, None) == abi.HPRMS_E_INVALID
    assert L.hprms_rmsnorm(0x1000, 0x2000, 0x3000, 4, 64, 63, 64, 0, 1e-6, None) == abi.HPRMS_E_INVALID


def test_errors_are_thread_local():
    import threading
    assert fused(dtype=9) == abi.HPRMS_E_INVALID
    seen = {}

    def other():
        seen["msg"] = abi.last_error()
    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["msg"] == ""
    assert "dtype" in abi.last_error()


def entry_points_find_kernels(L, hidden, dtype, base):
    """Every entry point with rows = 0 validates and looks its kernel up without
    launching; `base` 0 gives 128-byte aligned rows, 2 rows at a 2-byte boundary
    (the unaligned and tail variants)."""
    x, w, r, o, ro = base, base, base, base, base
    h = hidden
    assert L.hprms_fused_add_rmsnorm(x, w, r, 0, h, h, h, dtype, 1e-6, None) == abi.HPRMS_OK, abi.last_error()
    assert L.hprms_rmsnorm(o, x, w, 0, h, h, h, dtype, 1e-6, None) == abi.HPRMS_OK, abi.last_error()
    rc = L.hprms_fused_add_rmsnorm_fp8(o, 0, x, w, r, 0, h, h, h, h, dtype, 1e-6, None)
    assert rc == abi.HPRMS_OK, (h, abi.last_error())
    rc = L.hprms_fused_add_rmsnorm_out(o, ro, x, w, r, 0, h, h, h, h, h, dtype, 1e-6, None)
    assert rc == abi.HPRMS_OK, (h, abi.last_error())
    rc = L.hprms_reduce_add_rmsnorm(o, None, 2, w, r, 0, h, h, h, h, dtype, 1e-6, None)
    assert rc == abi.HPRMS_OK, (h, abi.last_error())
    for fmt, qw in ((abi.MX_FP8_E4M3, h), (abi.MX_FP4_E2M1, h // 2)):
        rc = L.hprms_fused_add_rmsnorm_mx(o, 0, x, w, r, 0, h, qw, h // 32, h, h, fmt, dtype, 1e-6, None)
        want = abi.HPRMS_OK if h % 32 == 0 else abi.HPRMS_E_INVALID
        assert rc == want, (h, fmt, abi.last_error())


def test_wide_rows_at_1k_to_3k():
    """At 1K-3K and 1024 < rows <= 4096 the fused op in and out of place take
    32 lanes x ceil(H / 256) vectors, two rows per one-wave workgroup, except
    at 1K-2K where the table's 64 x 4 (four rows per workgroup) comes out in
    even rounds over the 256 CUs at up to 3072 rows, and past 2.5K in place
    at up to 1536 rows; the other forms, other row counts and widths past 3K
    keep the table's rows."""
    bf = abi.DTYPE_BF16
    every = (1280, 1536, 1792, 2048, 2304, 2560, 3072, 3584, 4096)
    wide = {1032: (1280, 1536, 2304, 2560, 3584, 4096), 2048: (1280, 1536, 2304, 2560, 3584, 4096),
            2056: every, 2560: every, 2816: every, 3072: every}
    for hidden, rows_wide in wide.items():
        for rows in (512, 1024) + every + (5120, 8192):
            for mode in (abi.MODE_FUSED, abi.MODE_OUT):
                c = abi.select_config(rows, hidden, bf, mode)
                # past 2.5K the in-place op starts above 1536 rows
                if rows in rows_wide and not (hidden > 2560 and mode == abi.MODE_FUSED and rows <= 1536):
                    assert (c.lanes_per_row, c.vec_per_lane, c.block_threads, c.flags & ~96) == \
                        (32, -(-hidden // 256), 64, 135), (hidden, rows, mode)
                else:
                    assert c.lanes_per_row != 32 or c.block_threads != 64, (hidden, rows, mode)
            for mode in (abi.MODE_PLAIN, abi.MODE_FP8, abi.MODE_REDUCE, abi.MODE_MXFP8):
                assert abi.select_config(rows, hidden, bf, mode).lanes_per_row != 32, (hidden, rows, mode)
    for mode in (abi.MODE_FUSED, abi.MODE_OUT):
        for hidden in (3080, 3584, 4096):
            assert abi.select_config(4096, hidden, bf, mode).lanes_per_row != 32


def test_wave_rows_at_3k_to_5k():
    """The fused op in and out of place and plain RMSNorm on rows on the
    128-byte grid at 3K-5K take one row per one-wave workgroup (64 lanes x ceil(H / 512) vectors)
    at 768 < rows <= 2048; rows off the grid, the other forms and other row
    counts keep the table."""
    for dtype in (abi.DTYPE_BF16, abi.DTYPE_FP16):
        for hidden in (3080, 3584, 4096, 4608, 5120):
            for rows in (769, 1024, 1536, 2048):
                for mode in (abi.MODE_FUSED, abi.MODE_OUT, abi.MODE_PLAIN):
                    c = abi.select_config(rows, hidden, dtype, mode)
                    assert c.as_tuple() == (1, 64, -(-hidden // 512), 0, 64, 0, 135), (hidden, rows, mode)
                    odd = abi.select_config(rows, hidden + 1, dtype, mode)   # off the grid
                    assert odd.block_threads != 64, (hidden, rows, mode)
                for mode in (abi.MODE_REDUCE, abi.MODE_FP8):
                    assert abi.select_config(rows, hidden, dtype, mode).block_threads != 64, (hidden, rows, mode)
            for rows in (300, 768, 2049):
                for mode in (abi.MODE_FUSED, abi.MODE_OUT, abi.MODE_PLAIN):
                    assert abi.select_config(rows, hidden, dtype, mode).block_threads != 64, (hidden, rows, mode)
        for hidden in (3072, 5128, 6144):
            assert abi.select_config(1024, hidden, dtype, abi.MODE_FUSED).lanes_per_row != 64


def test_pair_rows_at_5k_to_8k():
    """The fused op in and out of place on rows on the 128-byte grid at 5K-8K
    takes one row per two-wave workgroup (128 lanes x ceil(H / 1024) vectors)
    at 512 < rows <= 1280; rows off the grid, the other forms and other row
    counts keep the table."""
    for dtype in (abi.DTYPE_BF16, abi.DTYPE_FP16):
        for hidden in (5184, 6144, 7168, 8192):
            for rows in (513, 768, 1024, 1280):
                for mode in (abi.MODE_FUSED, abi.MODE_OUT):
                    c = abi.select_config(rows, hidden, dtype, mode)
                    assert c.as_tuple() == (1, 128, -(-hidden // 1024), 0, 128, 0, 135), (hidden, rows, mode)
                    assert abi.select_config(rows, hidden + 1, dtype, mode).block_threads != 128
                for mode in (abi.MODE_REDUCE, abi.MODE_PLAIN, abi.MODE_FP8):
                    assert abi.select_config(rows, hidden, dtype, mode).block_threads != 128, (hidden, rows, mode)
            for rows in (300, 512, 1281, 4096):
                for mode in (abi.MODE_FUSED, abi.MODE_OUT):
                    assert abi.select_config(rows, hidden, dtype, mode).block_threads != 128, (hidden, rows)


def ref_rows(rows, cus):
    """rows on `cus` CUs as the row count with as many rows per CU on 256"""
    return -(-rows * 256 // cus)


def test_row_rules_scale_with_the_cu_count():
    """The table's row-count rules at 32, 80 and 256 CUs: on C CUs a call of
    R rows takes what a 256-CU device gives ceil(R * 256 / C) rows (the wide
    rows' comparison of workgroup rounds aside, checked below), so the
    latency rows, one- and two-wave rows, wide rows and LDS-staged weight
    keep their rows per CU; at 256 CUs the choice is hprms_select_config's."""
    bf = abi.DTYPE_BF16
    hiddens = (512, 1024, 1032, 2048, 2056, 3072, 4096, 5120, 6144, 8192, 8191, 12289, 16384, 16391, 32768)
    rowss = (1, 8, 32, 100, 128, 129, 256, 300, 400, 512, 640, 768, 1000, 1024, 1280, 2048, 4096, 8192)
    for mode in range(8):
        for hidden in hiddens:
            if (mode >= 5 and hidden % 32) or (mode == 7 and hidden % 128):
                continue
            for rows in rowss:
                assert abi.select_config(rows, hidden, bf, mode, cus=256).as_tuple() == \
                    abi.select_config(rows, hidden, bf, mode).as_tuple(), (mode, hidden, rows)
                for cus in (32, 80):
                    r = ref_rows(rows, cus)
                    if mode in (0, 3) and 128 < hidden // 8 <= 256 and 1024 < r <= 3072:
                        continue   # workgroup rounds counted on the call's own CUs
                    assert abi.select_config(rows, hidden, bf, mode, cus=cus).as_tuple() == \
                        abi.select_config(r, hidden, bf, mode).as_tuple(), (mode, hidden, rows, cus)
    # the fused op's latency rows at H = 1024 end at 1024 rows on 256 CUs, 128 on 32
    lat = abi.select_config(1, 1024, bf, 0).as_tuple()
    assert abi.select_config(128, 1024, bf, 0, cus=32).as_tuple() == lat
    assert abi.select_config(129, 1024, bf, 0, cus=32).as_tuple() != lat
    assert abi.select_config(1024, 1024, bf, 0).as_tuple() == lat
    # wide rows at 1K-2K where 64 x 4's rounds come out uneven on the device's CUs: on 80 CUs,
    # 400 rows are 3 rounds of two-row workgroups (6 rows per CU) against 2 of four-row ones (8)
    assert abi.select_config(400, 2048, bf, 0, cus=80).lanes_per_row == 32
    # 640 rows: 4 rounds of two-row workgroups and 2 of four-row ones, 8 rows per CU either way
    assert abi.select_config(640, 2048, bf, 0, cus=80).as_tuple() == abi.select_config(4096, 2048, bf, 0, cus=80).as_tuple()
    assert abi.select_config(640, 2048, bf, 0, cus=80).lanes_per_row == 64
    # the weight staged in LDS (odd widths): from 1024 rows on 256 CUs, from 128 on 32
    assert not abi.select_config(127, 12289, bf, 0, cus=32).flags & 16384
    assert abi.select_config(128, 12289, bf, 0, cus=32).flags & 16384


def test_row_groups_in_runs_per_xcd_at_two_pitches():
    """The in-place op takes its row groups in runs per XCD (flags bits 16-18)
    at H = 4096 from 4096 rows (runs of 32) and H = 8192 from 2048 rows (runs
    of 64), in both dtypes, on the table's shape; no other mode, width or row
    count, and no variant for rows off the grid, takes them."""
    for dtype in (abi.DTYPE_BF16, abi.DTYPE_FP16):
        for hidden, v, first in ((4096, 5, 4096), (8192, 6, 2048)):
            for rows in (first, first + 1, 3 * first, 16384):
                c = abi.select_config(rows, hidden, dtype)
                assert (c.flags >> 16) & 7 == v and c.flags & 0xffff == (131 if hidden == 4096 else 7), c.as_tuple()
            assert not abi.select_config(first - 1, hidden, dtype).flags >> 16
            for mode in range(1, 8):
                assert not abi.select_config(first, hidden, dtype, mode).flags >> 16, mode
            assert not abi.select_config(first, hidden + 1, dtype).flags >> 16   # odd width: the tail variant
        for hidden in (1024, 2048, 3072, 5120, 6144, 7168, 9216, 12288, 16384, 24576, 28672, 32768):
            for rows in (2048, 4096, 16384):
                assert not abi.select_config(rows, hidden, dtype).flags >> 16, (hidden, rows)
    # on 32 CUs the row counts scale: H = 8192 from 256 rows
    assert (abi.select_config(256, 8192, abi.DTYPE_BF16, cus=32).flags >> 16) & 7 == 6
    assert not abi.select_config(255, 8192, abi.DTYPE_BF16, cus=32).flags >> 16


@pytest.mark.parametrize("cus", [0, -1, 65537])
def test_select_config_cu_rejects_bad_cu_counts(cus):
    c = abi.Config()
    assert abi.lib().hprms_select_config_cu(4096, 4096, abi.DTYPE_BF16, 0, cus, ctypes.byref(c)) == abi.HPRMS_E_INVALID
    assert "cu_count" in abi.last_error()


def test_tail_weight_staged_in_lds_from_a_row_count():
    """The tail variants of 512 x 2-4 and 1024 x 2-3 stage the weight in LDS
    (flags bit 14) from 1024 rows (plain RMSNorm: 384), never in 1024 x 4, the
    fused op's 1024 x 3, the partial sums' 1024 x 2, the FP8 output or the
    variants without the tail."""
    bf = abi.DTYPE_BF16
    for hidden in (8191, 12289, 16391):
        assert not abi.select_config(1023, hidden, bf, 0).flags & 16384
        assert abi.select_config(1024, hidden, bf, 0).flags & 16384
        assert abi.select_config(1024, hidden, bf, 3).flags & 16384
        assert not abi.select_config(4096, hidden, bf, 2).flags & 16384
    assert not abi.select_config(383, 16391, bf, 1).flags & 16384
    assert abi.select_config(384, 16391, bf, 1).flags & 16384
    assert abi.select_config(4096, 12289, bf, 4).flags & 16384
    assert not abi.select_config(4096, 16391, bf, 4).flags & 16384       # 1024 x 2
    assert not abi.select_config(4096, 20479, bf, 0).flags & 16384       # 1024 x 3
    assert abi.select_config(4096, 20479, bf, 1).flags & 16384
    assert not abi.select_config(4096, 32775, bf, 0).flags & 16384       # 1024 x 4
    for hidden in (8192, 12288, 16384):
        assert not abi.select_config(4096, hidden, bf, 0).flags & 16384  # no tail


def test_table_covers_every_hidden_with_a_built_kernel():
    """Every hidden size maps either to a built vector-tier kernel that covers
    it, or (hidden < 8 or > 65543) to the general kernel; the choice for rows
    off the 128-byte grid has its unaligned and tail variants built; checked
    through the entry points with rows = 0 (they validate and look the kernel
    up, and launch nothing)."""
    L = abi.lib()
    built = {(dt, m): {c.as_tuple() for c in abi.kernel_configs(dt, m)}
             for dt in (abi.DTYPE_BF16, abi.DTYPE_FP16) for m in range(8)}
    for dtype, rows in ((abi.DTYPE_BF16, 4096), (abi.DTYPE_FP16, 4096), (abi.DTYPE_BF16, 1), (abi.DTYPE_FP16, 256)):
        for hidden in list(range(8, 70000, 8)) + [1, 3, 7, 9, 15, 1001, 4097, 65535, 65537, 65543, 65545]:
            c = abi.select_config(rows, hidden, dtype)
            if hidden < 8 or hidden // 8 > 8192:   # the table's last row holds 8192 whole vectors
                assert c.tier == 3
                continue
            assert c.tier in (1, 2)
            assert (c.flags & 96) == (96 if hidden % 8 else 0)
            assert c.lanes_per_row * c.vec_per_lane >= hidden // 8
            assert c.block_threads % c.lanes_per_row == 0
            for mode in range(8):
                if (mode >= 5 and hidden % 32) or (mode == 7 and hidden % 128):
                    continue
                cm = abi.select_config(rows, hidden, dtype, mode)
                t = cm.as_tuple()
                assert t in built[(dtype, mode)], (hidden, mode, t)
                # the choice for rows off the grid (odd widths report it: the tail
                # variant, with the sc1 bits the dispatch keeps) in its unaligned and
                # tail variants, with and without sc1; rows off the grid keep the default
                # row-group order (no runs per XCD, bits 16-18)
                hw = hidden + (1 if hidden % 8 == 0 and mode <= 4 else 0)
                off = abi.select_config(rows, hw, dtype, mode).as_tuple()
                u = (off[6] & ~(24 | 64 | 16384 | (7 << 16))) | 32
                if mode in (0, 3, 4) and off[1] == 1024 and off[2] in (2, 3):
                    u &= ~4   # the weight loaded late by the tail variant only
                assert off[:6] + (u,) in built[(dtype, mode)], (hidden, mode, off)
                if mode <= 4:
                    assert off[6] & 96 == 96, (hidden, mode, off)
                    if mode == 2 or rows * hw <= 1 << 24 or hw // 8 <= 2048:
                        assert off[6] & 24 == 0, (hidden, mode, off)
                    assert off in built[(dtype, mode)], (hidden, mode, off)
                    us = ((off[6] & ~(64 | 16384)) | 32) & ~4 | (u & 4)   # with sc1, the weight as in u
                    assert off[:6] + (us,) in built[(dtype, mode)], (hidden, mode, off)
                    assert off[:6] + ((off[6] & ~24) | 96,) in built[(dtype, mode)], (hidden, mode, off)
            if hidden % 8 == 0 and hidden % 32 and hidden > 1024 and hidden not in (4104, 16392, 65528):
                continue   # the lookups are exercised at every size class below and at the odd sizes
            entry_points_find_kernels(L, hidden, dtype, 0)
            entry_points_find_kernels(L, hidden, dtype, 2)
            if hidden % 8 == 0:
                rc = L.hprms_fused_add_rmsnorm_config(0, 0, 0, 0, hidden, hidden, hidden, dtype, 1e-6,
                                                      ctypes.byref(c), None)
                assert rc == abi.HPRMS_OK, (hidden, c.as_tuple(), abi.last_error())
                # the bench library also has the FP8 and partial-sum tables' choices as
                # fused (mode 0) kernels, so the 16-bit op can be run with the same lane
                # mapping (the partial sums' part prefetch has no in-place form; the tests
                # run it in the default row-group order, which changes no row's result)
                for other in (2, 4):
                    c8 = abi.select_config(rows, hidden, dtype, other)
                    c8.flags &= ~(32768 | (7 << 16))
                    assert c8.lanes_per_row * c8.vec_per_lane * 8 >= hidden
                    rc = abi.BENCH.lib().hprms_fused_add_rmsnorm_config(0, 0, 0, 0, hidden, hidden, hidden,
                                                                        dtype, 1e-6, ctypes.byref(c8), None)
                    assert rc == abi.HPRMS_OK, (hidden, other, c8.as_tuple(), abi.BENCH.last_error())


def test_config_entry_rejects_unbuilt_and_misfit_configs():
    L = abi.lib()
    c = abi.Config(1, 128, 3, 0, 256, 0, 3)  # not instantiated
    assert L.hprms_fused_add_rmsnorm_config(0, 0, 0, 0, 3072, 3072, 3072, 0, 1e-6, ctypes.byref(c),
                                            None) == abi.HPRMS_E_INVALID
    assert "no kernel built" in abi.last_error()
    c = abi.Config(1, 64, 1, 0, 256, 0, 3)   # covers 512 elements only
    assert L.hprms_fused_add_rmsnorm_config(0, 0, 0, 0, 4096, 4096, 4096, 0, 1e-6, ctypes.byref(c),
                                            None) == abi.HPRMS_E_INVALID
    assert "does not fit" in abi.last_error()


def test_every_built_config_is_well_formed():
    for dtype in (abi.DTYPE_BF16, abi.DTYPE_FP16):
        for mode in range(8):
            cfgs = abi.kernel_configs(dtype, mode)
            assert cfgs
            for c in cfgs:
                assert c.lanes_per_row in (16, 32, 64, 128, 256, 512, 1024)
                assert c.block_threads % 64 == 0 and c.block_threads % c.lanes_per_row == 0
                assert 0 <= c.lds_vec_per_lane <= c.vec_per_lane
                assert c.tier == (2 if c.lds_vec_per_lane else 1)
                # LDS spill of a workgroup fits the 160 KiB of a gfx950 CU
                assert c.lds_vec_per_lane * c.block_threads * 16 <= 160 * 1024


def test_fp8_entry_rejects_bad_arguments():
    L = abi.lib()
    ok = dict(out=0x4000, scale=0x5000, x=0x1000, w=0x2000, r=0x3000, so=4096)

    def call(**kw):
        a = dict(ok, **kw)
        return L.hprms_fused_add_rmsnorm_fp8(a["out"], a["scale"], a["x"], a["w"], a["r"], 4, 4096, a["so"],
                                             4096, 4096, 0, 1e-6, None)
    assert call(scale=0) == abi.HPRMS_E_INVALID and "null" in abi.last_error()
    assert call(out=0) == abi.HPRMS_E_INVALID
    assert call(so=100) == abi.HPRMS_E_INVALID and "output row stride" in abi.last_error()
    assert call(r=0x1000) == abi.HPRMS_E_INVALID and "alias" in abi.last_error()


def test_fp8_static_entry_rejects_bad_arguments():
    L = abi.lib()
    ok = dict(out=0x4000, scale=0x5000, x=0x1000, w=0x2000, r=0x3000, so=4096)

    def call(**kw):
        a = dict(ok, **kw)
        return L.hprms_fused_add_rmsnorm_fp8_static(a["out"], a["scale"], a["x"], a["w"], a["r"], 4, 4096, a["so"],
                                                    4096, 4096, 0, 1e-6, None)
    assert call(scale=0) == abi.HPRMS_E_INVALID and "null" in abi.last_error()
    assert call(out=0) == abi.HPRMS_E_INVALID
    assert call(so=100) == abi.HPRMS_E_INVALID and "output row stride" in abi.last_error()
    assert call(r=0x1000) == abi.HPRMS_E_INVALID and "alias" in abi.last_error()
    # no rows: validated, nothing launched, null pointers allowed
    assert L.hprms_fused_add_rmsnorm_fp8_static(0, 0, 0, 0, 0, 0, 4096, 4096, 4096, 4096, 0, 1e-6,
                                                None) == abi.HPRMS_OK


def test_out_of_place_entry_rejects_bad_arguments():
    L = abi.lib()
    ok = dict(out=0x4000, ro=0x5000, x=0x1000, r=0x3000, w=0x2000, so=4096, sro=4096)

    def call(**kw):
        a = dict(ok, **kw)
        return L.hprms_fused_add_rmsnorm_out(a["out"], a["ro"], a["x"], a["r"], a["w"], 4, 4096, a["so"], a["sro"],
                                             4096, 4096, 0, 1e-6, None)
    assert call(ro=0x4000) == abi.HPRMS_E_INVALID and "alias" in abi.last_error()
    assert call(out=0x3000) == abi.HPRMS_E_INVALID and "alias" in abi.last_error()
    assert call(ro=0x1000) == abi.HPRMS_E_INVALID and "alias" in abi.last_error()
    assert call(out=0x1000, so=8192) == abi.HPRMS_E_INVALID and "strides" in abi.last_error()
    assert call(sro=100) == abi.HPRMS_E_INVALID and "residual output row stride" in abi.last_error()
    assert call(ro=0) == abi.HPRMS_E_INVALID and "null" in abi.last_error()
    # zero rows: a configuration check only, every pointer may be null
    assert L.hprms_fused_add_rmsnorm_out(0, 0, 0, 0, 0, 0, 4096, 4096, 4096, 4096, 4096, 0, 1e-6, None) == abi.HPRMS_OK


def test_reduce_entry_rejects_bad_arguments():
    L = abi.lib()
    parts = (ctypes.c_void_p * 8)(*[0x10000 * (g + 1) for g in range(8)])

    def call(out=0x100000, p=parts, n=2, res=0x200000, po=4096, sp=4096):
        return L.hprms_reduce_add_rmsnorm(out, p, n, 0x300000, res, 4, 4096, po, sp, 4096, 0, 1e-6, None)
    assert call(n=0) == abi.HPRMS_E_INVALID and "nparts" in abi.last_error()
    assert call(n=9) == abi.HPRMS_E_INVALID and "nparts" in abi.last_error()
    assert call(p=None) == abi.HPRMS_E_INVALID and "parts" in abi.last_error()
    assert call(res=0x20000) == abi.HPRMS_E_INVALID and "alias" in abi.last_error()
    assert call(out=0x200000) == abi.HPRMS_E_INVALID and "alias" in abi.last_error()
    assert call(out=0x10000, po=8192) == abi.HPRMS_E_INVALID and "stride" in abi.last_error()
    assert call(sp=100) == abi.HPRMS_E_INVALID and "row stride" in abi.last_error()
    holes = (ctypes.c_void_p * 2)(0x10000, None)
    assert call(p=holes) == abi.HPRMS_E_INVALID and "part 1" in abi.last_error()
    assert abi.select_config(4096, 4096, abi.DTYPE_BF16, abi.MODE_REDUCE).tier in (1, 2)


def test_plain_c_caller_compiles_links_and_runs(tmp_path):
    """The header is C99 and the library answers a C program (no torch, no
    device): tests/c_abi_caller.c, built with gcc."""
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not found")
    libdir = os.path.dirname(abi.KERNEL_LIB)
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    exe = str(tmp_path / "c_abi_caller")
    cmd = [gcc, "-std=c99", "-Wall", "-Wextra", "-Werror=implicit-function-declaration", "-D__HIP_PLATFORM_AMD__",
           f"-I{os.path.join(ROOT, 'include')}", f"-I{os.path.join(rocm, 'include')}",
           os.path.join(ROOT, "tests", "c_abi_caller.c"), f"-L{libdir}", "-lhprms", f"-Wl,-rpath,{libdir}",
           "-o", exe]
    p = subprocess.run(cmd, capture_output=True, text=True)
    assert p.returncode == 0, p.stderr[-2000:]
    p = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert p.returncode == 0 and "ok" in p.stdout, p.stdout + p.stderr


def test_gpu_c_caller_is_built_and_links():
    """tests/c_gpu_caller (built with the libraries) loads libhprms.so, the
    oracle and the HIP runtime; without a device it stops with status 2 and
    says so, before any case runs."""
    import subprocess
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is present: tests/test_gpu_c_caller.py runs the program there")
    exe = os.path.join(ROOT, "tests", "c_gpu_caller")
    assert os.path.exists(exe), "tests/c_gpu_caller is not built: run __graft_entry__.build()"
    p = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert p.returncode == 2 and "case " not in p.stdout, p.stdout + p.stderr
    assert "hipGetDeviceCount" in p.stderr or "no HIP device" in p.stderr, p.stderr


def test_fp8_group_entry_rejects_bad_arguments():
    L = abi.lib()
    ok = dict(out=0x4000, sc=0x5000, x=0x1000, w=0x2000, r=0x3000, h=4096, so=4096, ss=32, gs=1)

    def call(**kw):
        a = dict(ok, **kw)
        return L.hprms_fused_add_rmsnorm_fp8_group(a["out"], a["sc"], a["x"], a["w"], a["r"], a.get("rows", 4),
                                                   a["h"], a["so"], a["ss"], a["gs"], a["h"], a["h"], 0, 1e-6, None)
    assert call(h=4160, so=4160, ss=33) == abi.HPRMS_E_INVALID and "128" in abi.last_error()
    assert call(so=2048) == abi.HPRMS_E_INVALID and "output row stride" in abi.last_error()
    # scale strides that lay the scales out neither as rows nor as columns: rows of scales
    # that overlap, groups that collide, columns (rows = 4) that overlap, and (3, 8), which
    # interleaves rows and groups without a collision
    for ss, gs in ((31, 1), (0, 1), (32, 0), (62, 2), (1, 3), (2, 6), (1, 1), (3, 8)):
        assert call(ss=ss, gs=gs) == abi.HPRMS_E_INVALID and "neither as rows" in abi.last_error(), (ss, gs)
    for ss, gs in ((-1, 1), (32, -1), (32, 1 << 41), (1 << 41, 1)):
        assert call(ss=ss, gs=gs) == abi.HPRMS_E_INVALID and "out of range" in abi.last_error(), (ss, gs)
    # one row, or one group: the other stride is free
    assert call(rows=0, ss=0, gs=0, h=128, so=128) == abi.HPRMS_OK
    # a row group's scales must fit one buffer resource (H = 128: 64 rows per workgroup,
    # the column-major group stride spans 2^29 floats)
    assert call(rows=0, h=256, so=256, ss=1, gs=1 << 29) == abi.HPRMS_E_INVALID and "2 GiB" in abi.last_error()
    assert call(rows=0, h=256, so=256, ss=1, gs=1 << 20) == abi.HPRMS_OK
    assert call(sc=0) == abi.HPRMS_E_INVALID and "null" in abi.last_error()
    assert call(sc=0x5002) == abi.HPRMS_E_INVALID and "4-byte aligned" in abi.last_error()
    # outputs and rows off the 16-byte grid take the unaligned variants; odd addresses are refused
    assert call(out=0x4002, rows=0) == abi.HPRMS_OK and call(x=0x1008, rows=0) == abi.HPRMS_OK
    assert call(x=0x1001) == abi.HPRMS_E_INVALID and "aligned" in abi.last_error()
    # every width the form accepts maps to a vector-tier shape whose 128-element groups are
    # 16 adjacent lanes
    for hidden in range(128, 65536 + 1, 128):
        for rows in (1, 300, 1024, 4096):
            c = abi.select_config(rows, hidden, abi.DTYPE_BF16, abi.MODE_FP8_GROUP)
            assert c.tier in (1, 2) and c.lanes_per_row % 16 == 0, (hidden, rows, c.as_tuple())


def test_mx_entry_rejects_bad_arguments():
    L = abi.lib()
    ok = dict(out=0x4000, sc=0x5000, x=0x1000, w=0x2000, r=0x3000, h=4096, so=2048, ss=128, fmt=abi.MX_FP4_E2M1)

    def call(**kw):
        a = dict(ok, **kw)
        return L.hprms_fused_add_rmsnorm_mx(a["out"], a["sc"], a["x"], a["w"], a["r"], a.get("rows", 4), a["h"],
                                            a["so"], a["ss"], a["h"], a["h"], a["fmt"], 0, 1e-6, None)
    assert call(fmt=2) == abi.HPRMS_E_INVALID and "format" in abi.last_error()
    assert call(h=4104, so=4104, ss=200) == abi.HPRMS_E_INVALID and "32" in abi.last_error()
    assert call(so=1024) == abi.HPRMS_E_INVALID and "output row stride" in abi.last_error()
    assert call(fmt=abi.MX_FP8_E4M3) == abi.HPRMS_E_INVALID          # MXFP8 rows are hidden bytes wide
    assert call(ss=64) == abi.HPRMS_E_INVALID and "scale row stride" in abi.last_error()
    assert call(sc=0) == abi.HPRMS_E_INVALID and "null" in abi.last_error()
    # outputs and rows off the 16-byte grid take the unaligned variants; odd addresses are refused
    assert call(out=0x4002, rows=0) == abi.HPRMS_OK and call(x=0x1008, rows=0) == abi.HPRMS_OK
    assert call(x=0x1001) == abi.HPRMS_E_INVALID and "aligned" in abi.last_error()
    # a scale row stride whose row group would not fit one buffer resource is refused, not truncated
    # (H = 256 maps 8 rows to a workgroup)
    assert L.hprms_fused_add_rmsnorm_mx(0, 0, 0, 0, 0, 0, 256, 128, 1 << 29, 256, 256, abi.MX_FP4_E2M1, 0, 1e-6,
                                        None) == abi.HPRMS_E_INVALID
    assert "2 GiB" in abi.last_error()
    assert L.hprms_fused_add_rmsnorm_mx(0, 0, 0, 0, 0, 0, 256, 128, 1 << 20, 256, 256, abi.MX_FP4_E2M1, 0, 1e-6,
                                        None) == abi.HPRMS_OK
    # the vector kernels take 32-bit input and residual row strides, also with one row per workgroup
    assert L.hprms_fused_add_rmsnorm_mx(0, 0, 0, 0, 0, 0, 32768, 32768, 1024, 1 << 31, 32768, abi.MX_FP4_E2M1, 0,
                                        1e-6, None) == abi.HPRMS_E_INVALID
    assert "2^31" in abi.last_error()
    assert L.hprms_fused_add_rmsnorm_mx(0, 0, 0, 0, 0, 0, 32768, 32768, 1024, (1 << 31) - 8, 32768,
                                        abi.MX_FP4_E2M1, 0, 1e-6, None) == abi.HPRMS_OK
    for mode in (abi.MODE_MXFP8, abi.MODE_MXFP4):
        c = abi.select_config(4096, 4096, abi.DTYPE_BF16, mode)
        assert c.tier in (1, 2) and c.lanes_per_row % 4 == 0


def test_latency_rows_end_at_the_per_mode_limits():
    """The latency rows take calls up to a per-mode, per-width row count; the
    next row count takes the bandwidth table (the same choice as 4096 rows, or
    as 8192 rows where 4096 rows take the wide rows of 1K-3K, in the default
    row-group order), or, in place at 3K-5K, one row per one-wave workgroup."""
    fp8_mx = {1024: 1024, 2048: 768, 4096: 768, 8192: 256, 16384: 256}
    limits = {abi.MODE_FUSED: {1024: 1024, 2048: 768, 4096: 768, 8192: 256, 16384: 384},
              abi.MODE_PLAIN: {1024: 1024, 2048: 256, 4096: 768, 8192: 256, 16384: 256},
              abi.MODE_FP8: fp8_mx, abi.MODE_MXFP8: fp8_mx, abi.MODE_MXFP4: fp8_mx,
              abi.MODE_OUT: {h: 256 for h in fp8_mx}, abi.MODE_REDUCE: {h: 256 for h in fp8_mx}}
    for mode, by_hidden in limits.items():
        for hidden, limit in by_hidden.items():
            for dtype in (abi.DTYPE_BF16, abi.DTYPE_FP16):
                lat = abi.select_config(1, hidden, dtype, mode).as_tuple()
                assert abi.select_config(limit, hidden, dtype, mode).as_tuple() == lat, (mode, hidden)
                past = abi.select_config(limit + 1, hidden, dtype, mode).as_tuple()
                want = abi.select_config(4096, hidden, dtype, mode)
                if (want.lanes_per_row, want.block_threads) == (32, 64):
                    want = abi.select_config(8192, hidden, dtype, mode)
                if mode in (abi.MODE_FUSED, abi.MODE_OUT, abi.MODE_PLAIN) and 3072 < hidden <= 5120 \
                        and limit >= 768:
                    want = abi.Config(1, 64, hidden // 512, 0, 64, 0, 135)
                want.flags &= ~(7 << 16)   # (row groups in runs per XCD only from 2048 rows)
                assert past == want.as_tuple(), (mode, hidden)


def test_bench_library_is_apart_from_the_product():
    """libhprms_bench.so carries the same C ABI plus the tuning-only kernel
    shapes and the ceiling / timeline entry points; libhprms.so exports none
    of those and holds only shapes the dispatch tables can choose."""
    bench = abi.BENCH.lib()
    for n in declared_functions():
        assert hasattr(bench, n), n
    extra = ("hprms_bench_fused_timeline", "hprms_bench_form_config", "hprms_ceil_empty", "hprms_ceil_read",
             "hprms_ceil_write", "hprms_ceil_copy", "hprms_ceil_skeleton", "hprms_ceil_streams", "hprms_ceil_flat")
    for n in extra:
        assert hasattr(bench, n), n
        assert not hasattr(abi.lib(), n), f"{n} must not be in the product library"
    for mode in range(8):
        for dt in (abi.DTYPE_BF16, abi.DTYPE_FP16):
            prod = {c.as_tuple() for c in abi.kernel_configs(dt, mode)}
            more = {c.as_tuple() for c in abi.BENCH.kernel_configs(dt, mode)}
            assert prod <= more
    tuning = {c.as_tuple() for c in abi.BENCH.kernel_configs(abi.DTYPE_BF16, 0)} - \
        {c.as_tuple() for c in abi.kernel_configs(abi.DTYPE_BF16, 0)}
    assert (1, 128, 4, 0, 256, 0, 391) in tuning and (1, 1024, 4, 0, 1024, 0, 671) in tuning


def test_bench_entry_points_reject_bad_arguments():
    L = abi.BENCH.lib()
    assert L.hprms_ceil_empty(0, 256, None) == abi.HPRMS_E_INVALID
    assert L.hprms_ceil_empty(4, 96, None) == abi.HPRMS_E_INVALID
    assert L.hprms_ceil_flat(1, 256, 3, 0, 0x1000, 0x2000, 4096, None) == abi.HPRMS_E_INVALID   # no such shape
    assert L.hprms_ceil_flat(1, 256, 1, 0, 0x1000, 0x2008, 4096, None) == abi.HPRMS_E_INVALID   # misaligned
    assert L.hprms_ceil_flat(1, 256, 1, 0, 0x1000, 0x2000, 1 << 30, None) == abi.HPRMS_E_INVALID
    assert L.hprms_ceil_copy(0x1000, 0x2008, 4096, None) == abi.HPRMS_E_INVALID   # misaligned source
    assert L.hprms_ceil_read(0x1000, 0x2000, 4095, 0x3000, None) == abi.HPRMS_E_INVALID
    assert L.hprms_ceil_skeleton(0x1000, 0x2000, 4, 4096, 128, 3, 256, 3, None) == abi.HPRMS_E_INVALID
    assert L.hprms_ceil_skeleton(0x1000, 0x2000, 4, 4096, 128, 4, 256, 7, None) == abi.HPRMS_E_INVALID
    c = abi.Config(1, 128, 4, 0, 256, 0, 643)
    assert L.hprms_bench_fused_timeline(0x1000, 0x2000, 0x3000, 4, 4096, abi.DTYPE_BF16, 1e-6, ctypes.byref(c),
                                        None, None) == abi.HPRMS_E_INVALID
    # a timeline configuration through the ordinary forced-config entry has no buffer to write
    assert abi.BENCH.lib().hprms_fused_add_rmsnorm_config(0x1000, 0x2000, 0x3000, 4, 4096, 4096, 4096,
                                                          abi.DTYPE_BF16, 1e-6, ctypes.byref(c),
                                                          None) == abi.HPRMS_E_INVALID
    assert "timeline" in abi.BENCH.last_error()
    # the other forms with a forced configuration: modes 1, 2, 3, 5, 6, 7 only, a built shape,
    # and mode 7's scale layout checked as in the product entry (rows = 0 launches nothing)
    q = abi.Config(1, 512, 2, 0, 512, 0, 7 | 5 << 16)
    rest = (0x1000, 0x2000, 0x3000, 0, 8192, abi.DTYPE_BF16, 1e-6)
    for mode, ss, gs in ((2, 0, 0), (5, 256, 1), (6, 256, 1), (7, 1, 64), (7, 64, 1), (3, 0, 0)):
        rc = L.hprms_bench_form_config(mode, 0x4000, 0x5000, ss, gs, *rest, ctypes.byref(q), None)
        assert rc == abi.HPRMS_OK, (mode, abi.BENCH.last_error())
    args = (0x4000, 0x5000, 1, 64) + rest
    assert L.hprms_bench_form_config(0, *args, ctypes.byref(q), None) == abi.HPRMS_E_INVALID
    assert L.hprms_bench_form_config(4, *args, ctypes.byref(q), None) == abi.HPRMS_E_INVALID
    plain = abi.Config(1, 512, 2, 0, 512, 0, 31 | 6 << 16)
    assert L.hprms_bench_form_config(1, 0x4000, 0, 0, 0, *rest, ctypes.byref(plain), None) == abi.HPRMS_OK
    assert L.hprms_bench_form_config(7, *args, None, None) == abi.HPRMS_E_INVALID
    bad = abi.Config(1, 512, 2, 0, 512, 0, 7 | 3 << 16)
    assert L.hprms_bench_form_config(7, *args, ctypes.byref(bad), None) == abi.HPRMS_E_INVALID
    assert "no kernel built" in abi.BENCH.last_error()
    assert L.hprms_bench_form_config(7, 0x4000, 0x5000, 1, 1, *args[4:], ctypes.byref(q), None) == abi.HPRMS_OK
    assert L.hprms_bench_form_config(7, 0x4000, 0x5000, 1, -1, *args[4:], ctypes.byref(q), None) == \
        abi.HPRMS_E_INVALID


def _reachable(dtype, mode):
    """Every vector-tier kernel the dispatch tables can launch for (dtype,
    mode): at each width and at both sides of each latency row's row-count
    limit, the choice for rows on the 128-byte grid (aligned, and unaligned
    when sc1 is dropped for small calls) and the choice for rows off it
    (reported for odd widths, with the sc1 bits the dispatch keeps for calls
    past 16 Mi elements in modes 0, 1, 3 and 4) in its unaligned and (modes
    0-4) tail variants, which take their row groups in the default order."""
    out = set()
    for rows in (1, 256, 257, 384, 385, 768, 769, 1024, 1025, 4096):
        for nvec in range(1, 8193):
            c = abi.select_config(rows, nvec * 8, dtype, mode)
            if c.tier == 3:
                continue
            shape = (c.tier, c.lanes_per_row, c.vec_per_lane, c.lds_vec_per_lane, c.block_threads, 0)
            out.add(shape + (c.flags,))
            if mode == 7 and nvec == 512 and rows >= 4096 and c.flags == 7 and shape[1:5] == (256, 2, 0, 256):
                out.add(shape + (7 | 5 << 16,))   # column-major scales at 8 KiB rows: runs of 32 per XCD
            c.flags &= ~(7 << 16)   # the variants keep the default row-group order
            if c.flags & 24:
                out.add(shape + ((c.flags & ~24) | 32,))
            if mode <= 4:
                t = abi.select_config(rows, nvec * 8 + 1, dtype, mode)   # off the grid: its tail variant
                tshape = (t.tier, t.lanes_per_row, t.vec_per_lane, t.lds_vec_per_lane, t.block_threads, 0)
                out.add(tshape + (t.flags,))
                # its unaligned sibling; in 1024 x 2 and x 3 only the tail loads the weight late
                # in modes 0, 3 and 4
                u = t.flags & ~(64 | 16384)   # (only tails stage the weight in LDS)
                if mode in (0, 3, 4) and t.lanes_per_row == 1024 and t.vec_per_lane in (2, 3):
                    u &= ~4
                out.add(tshape + (u,))
                # rows of this width off the grid: the rotated variant keeps sc1 past 16 Mi
                # elements (the rows with sc1 bits take the same shape on and off the grid)
                if mode != 2 and c.flags & 24 and rows * nvec * 8 > 1 << 24:
                    out.add(shape + (c.flags | 32,))
            else:
                out.add(shape + ((c.flags & ~24) | 32,))
    return out


def test_product_library_holds_exactly_the_reachable_kernels():
    """libhprms.so instantiates the kernels its tables can choose and no
    other (the tuning shapes live in the bench library)."""
    for dtype in (abi.DTYPE_BF16, abi.DTYPE_FP16):
        for mode in range(8):
            built = {c.as_tuple() for c in abi.kernel_configs(dtype, mode)}
            assert built == _reachable(dtype, mode), (dtype, mode, sorted(built ^ _reachable(dtype, mode)))
