"""GPU parity of the vector tiers' variants for rows off the 128-byte grid.

The dispatch (hprms.hip, needs_unaligned / shift_rows) sends rows that do not
all start on a 128-byte boundary to a variant of the table's shape:
  * hidden % 8 == 0: the unaligned variant (flags bit 5: rows at any 2-byte
    boundary, no sc1 bits), which keeps the shape's arithmetic; on rows whose
    written stream is 16-byte aligned it rotates each row's lane mapping so
    that every wave's 1 KiB access starts on a 512-byte boundary (the first
    up to 31 lanes take the row's last vectors), so its sum of squares runs in another
    order there and its output is held to the oracle's bar, its residual to
    the aligned kernel's bits; on rows that are not rotated it gives the same
    bits as the table's kernel on contiguous aligned copies;
  * hidden % 8 != 0: the tail variant (bit 6), whose lane holding the last
    whole vector also handles the 16 bytes that end at the row's end;
  * from 513 whole vectors up, modes 0-4 whose streams (the weight aside)
    are all off 16-byte alignment: the tail variant with shifted rows, which
    starts each row's body vectors at the first written stream's first
    16-byte boundary and adds a head vector for the elements before them; its
    sum of squares runs in another order, so its output is held to the
    oracle's bar and its residual to the same bits.
Every mode is within the usual bar of the oracle (residual bit-exact, 16-bit
output within 1 ulp, FP8 within 1 e4m3 ulp) and writes nothing outside the
views; the edge vectors are exercised at both ends of every table row, at
every tail length 1-7, on the latency rows and next to the limits.
"""
import numpy as np
import pytest
import torch

from helpers import DT, assert_output_close, assert_residual_exact, bits, make_inputs, oracle_fused
from oracle import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
EPS = 1e-6
# whole vectors (8 elements) held by each row of the fused table (hprms.hip, table_config)
TABLE_NVEC = [16, 32, 64, 128, 256, 384, 512, 1024, 1536, 2047, 2048, 3072, 4096, 8192]


@pytest.fixture(scope="module")
def abi():
    assert torch.cuda.is_available(), "the gpu tests need a HIP device"
    import hp_rms_norm_amd  # noqa: F401  (fails loudly if unbuilt)
    from hp_rms_norm_amd import abi as a
    a.lib()
    return a


def _stream():
    return torch.cuda.current_stream().cuda_stream


class View:
    """A [rows, hidden] view at element offset `off` of a [rows, off + hidden +
    pad] device buffer filled with `fill`; the buffer is kept to check that
    nothing outside the view is written."""

    def __init__(self, t, off, pad, fill=0x5A5A):
        rows, hidden = t.shape
        self.buf = torch.full((rows, off + hidden + pad), 0, dtype=torch.int16, device=DEV)
        self.buf.fill_(fill - 65536 if fill > 32767 else fill)
        self.buf = self.buf.view(t.dtype)
        self.view = self.buf[:, off:off + hidden]
        self.view.copy_(t.to(DEV))
        self.off, self.hidden = off, hidden
        self.outside = self._outside()

    def _outside(self):
        b = self.buf.view(torch.int16).cpu()
        return torch.cat([b[:, :self.off], b[:, self.off + self.hidden:]], 1).clone()

    @property
    def ptr(self):
        return self.view.data_ptr()

    @property
    def stride(self):
        return self.buf.shape[1]

    def check_outside(self, what):
        assert torch.equal(self._outside(), self.outside), f"{what}: wrote outside the view"


class ByteView:
    """The same for byte rows (quantised outputs, MX scales)."""

    def __init__(self, rows, width, off, pad):
        self.buf = torch.full((rows, off + width + pad), 0xA5, dtype=torch.uint8, device=DEV)
        self.view = self.buf[:, off:off + width]
        self.off, self.width = off, width

    @property
    def ptr(self):
        return self.view.data_ptr()

    @property
    def stride(self):
        return self.buf.shape[1]

    def check_outside(self, what):
        b = self.buf.cpu()
        assert bool((b[:, :self.off] == 0xA5).all()) and bool((b[:, self.off + self.width:] == 0xA5).all()), \
            f"{what}: wrote outside the view"


def u16(t):
    return t.detach().cpu().contiguous().view(torch.int16)


# ---- mode 0: the fused op in place ----------------------------------------------------------
def fused(abi, x, r, w, off=0, pad=0, woff=0, config=None):
    xv, rv, wv = View(x, off, pad), View(r, off + 3 if off else 0, pad), View(w[None], woff, 0)
    abi.fused_add_rmsnorm(xv.ptr, wv.ptr, rv.ptr, x.shape[0], x.shape[1], xv.stride, rv.stride, DT[x.dtype], EPS,
                          _stream(), config)
    torch.cuda.synchronize()
    xv.check_outside("input")
    rv.check_outside("residual")
    return u16(xv.view), u16(rv.view)


def widths_at_both_ends(tail):
    """Per table row: its smallest and largest width (with a tail of 1 and 7
    elements when `tail`, else whole vectors)."""
    out, lo = [], 0
    for hi in TABLE_NVEC:
        out += [8 * (lo + 1) + 1, 8 * hi + 7] if tail else [8 * (lo + 1), 8 * hi]
        lo = hi
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_misaligned_rows_equal_the_aligned_kernel_every_table_row(abi, dtype):
    """Rows 16-byte aligned off the 128-byte grid (stride hidden + 8, so the
    rows take every 16-byte phase and every rotation): the same residual bits
    as contiguous aligned tensors and the oracle's bar for the output.  Rows
    at a 2-byte offset with a row stride of hidden + 3 (and the weight off by
    one element): the same residual bits and the oracle's bar for the
    output."""
    for hidden in widths_at_both_ends(tail=False):
        for rows in (67, 3):
            x, r, w = make_inputs(rows, hidden, dtype, seed=hidden + rows)
            print("misaligned rows", rows, hidden, dtype, flush=True)
            want_out, want_res = fused(abi, x, r, w)
            o_out, o_res = oracle_fused(x, r, w, EPS, dtype)
            assert_residual_exact(want_res.numpy().view(np.uint16), o_res, dtype)
            assert_output_close(want_out.numpy().view(np.uint16), o_out, dtype)
            for off, pad, woff in ((1, 2, 1), (8, 0, 0)):
                got_out, got_res = fused(abi, x, r, w, off, pad, woff)
                tag = f"{rows}x{hidden} {dtype} off {off} pad {pad}"
                assert torch.equal(got_res, want_res), "residual differs from the aligned kernel " + tag
                assert_output_close(got_out.numpy().view(np.uint16), o_out, dtype, "output " + tag)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_tail_at_both_ends_of_every_table_row(abi, dtype):
    for hidden in widths_at_both_ends(tail=True):
        c = abi.select_config(67, hidden, DT[dtype])
        assert (c.flags & 96) == 96, (hidden, c.as_tuple())
        x, r, w = make_inputs(67, hidden, dtype, seed=hidden)
        print("tail", hidden, dtype, c.as_tuple(), flush=True)
        got_out, got_res = fused(abi, x, r, w)
        o_out, o_res = oracle_fused(x, r, w, EPS, dtype)
        tag = f"67x{hidden} {dtype}"
        assert_residual_exact(got_res.numpy().view(np.uint16), o_res, dtype, "residual " + tag)
        assert_output_close(got_out.numpy().view(np.uint16), o_out, dtype, "output " + tag)
        # the same rows at a 2-byte offset and padded (above 512 whole vectors each row is
        # shifted to its own 16-byte boundary)
        m_out, m_res = fused(abi, x, r, w, off=1, pad=5, woff=1)
        assert torch.equal(m_res, got_res), "misaligned tail rows, residual " + tag
        assert_output_close(m_out.numpy().view(np.uint16), o_out, dtype, "misaligned tail rows, output " + tag)


def test_every_tail_length_on_bandwidth_and_latency_rows(abi):
    """hidden = 4096 + t and 8192 + t, t = 1..7 (the tail overlaps the last
    whole vector by 8 - t elements; at 8192 + t rows are shifted and start at
    2t-byte steps, so the head and tail vectors take every length), on the
    bandwidth table (1100 rows) and the latency table (5 rows); outliers, so
    that every element's square matters."""
    for t in range(1, 8):
        for rows, hidden in ((1100, 4096 + t), (5, 4096 + t), (1100, 8192 + t), (5, 8192 + t)):
            for dtype in (torch.bfloat16, torch.float16):
                x, r, w = make_inputs(rows, hidden, dtype, seed=t + rows, dist="outliers")
                print("tail length", t, rows, dtype, flush=True)
                got_out, got_res = fused(abi, x, r, w)
                o_out, o_res = oracle_fused(x, r, w, EPS, dtype)
                tag = f"{rows}x{hidden} {dtype}"
                assert_residual_exact(got_res.numpy().view(np.uint16), o_res, dtype, "residual " + tag)
                assert_output_close(got_out.numpy().view(np.uint16), o_out, dtype, "output " + tag)


def test_tail_limits_and_special_values(abi):
    """The smallest widths with a tail (9 ... 15: the tail vector overlaps the
    only whole vector), the smallest with shifted rows (4104, 4105), the
    largest the vector tiers take (65543), and edge elements that are infinite
    or NaN (a masked duplicate must not turn an infinite sum of squares into
    NaN), on contiguous rows and at a 2-byte offset."""
    dtype = torch.bfloat16
    for hidden in (9, 10, 15, 16, 17, 4103, 4104, 4105, 65543):
        x, r, w = make_inputs(7, hidden, dtype, seed=hidden)
        print("tail limit", hidden, flush=True)
        got_out, got_res = fused(abi, x, r, w)
        o_out, o_res = oracle_fused(x, r, w, EPS, dtype)
        assert_residual_exact(got_res.numpy().view(np.uint16), o_res, dtype, f"residual {hidden}")
        assert_output_close(got_out.numpy().view(np.uint16), o_out, dtype, f"output {hidden}")
        m_out, m_res = fused(abi, x, r, w, off=1, pad=2, woff=1)
        assert_residual_exact(m_res.numpy().view(np.uint16), o_res, dtype, f"residual {hidden} off 1")
        assert_output_close(m_out.numpy().view(np.uint16), o_out, dtype, f"output {hidden} off 1")
    # 8195 elements (shifted rows): the tail vector is elements 8187 ... 8194; rows at
    # 16390-byte steps start 0, 3, 6, 1, 4, 7, 2, 5 elements past a 16-byte boundary, so
    # the head vector covers 0 ... 7 and its own elements are the first 8 - shift
    hidden = 8195
    x, r, w = make_inputs(8, hidden, dtype, seed=5)
    r[:] = 0
    x[0, 8194] = float("inf")      # element of the tail only
    x[1, 8188] = float("inf")      # in the tail's overlap: counted once, by its body vector
    x[2, 8193] = float("nan")
    x[3, 8187] = float("-inf")
    x[4, 0] = float("inf")         # element of the head only
    x[5, 7] = float("-inf")        # in the head's overlap
    x[6, 5] = float("nan")
    print("edge special values", flush=True)
    o_out, o_res = oracle_fused(x, r, w, EPS, dtype)
    for off, pad in ((0, 0), (1, 2)):
        got_out, got_res = fused(abi, x, r, w, off=off, pad=pad)
        assert_residual_exact(got_res.numpy().view(np.uint16), o_res, dtype, f"residual special off {off}")
        assert_output_close(got_out.numpy().view(np.uint16), o_out, dtype, f"output special off {off}")


# ---- rotated rows: every 16-byte phase, modes 0, 1, 3 and 4 ---------------------------------
# whole-vector widths around the table's rows; 48 has fewer than 8 vectors (not rotated),
# 1000 and 16376 end mid-line
ROT_WIDTHS = [48, 64, 1000, 1024, 4096, 5120, 8192, 12288, 16376, 16384, 24576, 32768]


@pytest.mark.parametrize("hidden", ROT_WIDTHS)
def test_rotated_rows_every_phase_every_mode(abi, hidden):
    """Written streams 16-byte aligned off the 128-byte grid: first elements at
    8j (j = 0 ... 7) and a row stride of 8j + hidden + 8 elements, so the rows
    take many 16-byte phases modulo 512 bytes (with j = 0 and hidden a multiple
    of 256, all 32 of them: every rotation of the lane mapping), on the bandwidth
    table (300 rows) and the latency table (5 rows); outliers so that every
    element's square matters; each mode against the oracle, and nothing
    written outside the views."""
    dtype = torch.bfloat16
    th = min(16, oracle.max_threads())
    for rows in (300, 5):
        x, r, w = make_inputs(rows, hidden, dtype, seed=hidden + rows, dist="outliers")
        o_out, o_res = oracle_fused(x, r, w, EPS, dtype)
        want_plain = oracle.rmsnorm(bits(x), bits(w), EPS, DT[dtype], threads=th)
        wd = w.to(DEV)
        for j in range(8):
            tag = f"{rows}x{hidden} phase {j}"
            print("rotated rows", tag, flush=True)
            xv, rv = View(x, 8 * j, 8), View(r, 8 * j, 8)
            abi.fused_add_rmsnorm(xv.ptr, wd.data_ptr(), rv.ptr, rows, hidden, xv.stride, rv.stride, DT[dtype],
                                  EPS, _stream())
            torch.cuda.synchronize()
            xv.check_outside("input " + tag)
            rv.check_outside("residual " + tag)
            assert_residual_exact(bits(rv.view), o_res, dtype, "fused residual " + tag)
            assert_output_close(bits(xv.view), o_out, dtype, "fused output " + tag)

            xa, ov = x.to(DEV), View(torch.zeros_like(x), 8 * j, 8)
            abi.rmsnorm(ov.ptr, xa.data_ptr(), wd.data_ptr(), rows, hidden, ov.stride, hidden, DT[dtype], EPS,
                        _stream())
            torch.cuda.synchronize()
            ov.check_outside("plain output " + tag)
            assert_output_close(bits(ov.view), want_plain, dtype, "plain " + tag)

            ra = r.to(DEV)
            ov, rov = View(torch.zeros_like(x), 8 * j, 8), View(torch.zeros_like(x), 8 * ((j + 3) % 8), 8)
            abi.fused_add_rmsnorm_out(ov.ptr, rov.ptr, xa.data_ptr(), ra.data_ptr(), wd.data_ptr(), rows, hidden,
                                      ov.stride, rov.stride, hidden, hidden, DT[dtype], EPS, _stream())
            torch.cuda.synchronize()
            ov.check_outside("out " + tag)
            rov.check_outside("residual_out " + tag)
            assert_residual_exact(bits(rov.view), o_res, dtype, "out residual " + tag)
            assert_output_close(bits(ov.view), o_out, dtype, "out output " + tag)

            # two parts, each x / 2, against the oracle's partial-sum form
            half = (x.float() / 2).to(dtype)
            parts = [half.to(DEV), half.to(DEV)]
            rv, ov = View(r, 8 * j, 8), View(torch.zeros_like(x), 8 * j, 8)
            abi.reduce_add_rmsnorm(ov.ptr, [p.data_ptr() for p in parts], wd.data_ptr(), rv.ptr, rows, hidden,
                                   ov.stride, hidden, rv.stride, DT[dtype], EPS, _stream())
            torch.cuda.synchronize()
            ov.check_outside("reduce output " + tag)
            rv.check_outside("reduce residual " + tag)
            p_out, p_res = oracle.reduce_add_rmsnorm([bits(half), bits(half)], bits(w), bits(r), EPS, DT[dtype],
                                                     threads=th)
            assert_residual_exact(bits(rv.view), p_res, dtype, "reduce residual " + tag)
            assert_output_close(bits(ov.view), p_out, dtype, "reduce output " + tag)


# calls past 16 Mi elements: the rotated variants keep the table row's sc1 bits (the tail
# variants on the 1024-lane rows past 2048 vectors only)
@pytest.mark.parametrize("hidden,off,pad", [(16384, 8, 0), (24576, 1, 8), (32775, 0, 0)])
def test_large_off_grid_calls_every_rotated_mode(abi, hidden, off, pad):
    """1100 rows (past 16 Mi elements) 16 bytes off the grid, 2 bytes off
    (shifted) and of an odd width: modes 0, 1, 3 and 4 against the oracle, and
    nothing written outside the views."""
    dtype, rows = torch.bfloat16, 1100
    th = min(16, oracle.max_threads())
    x, r, w = make_inputs(rows, hidden, dtype, seed=hidden + off)
    o_out, o_res = oracle_fused(x, r, w, EPS, dtype)
    wd = w.to(DEV)
    tag = f"{rows}x{hidden} off {off} pad {pad}"
    print("large off-grid call", tag, flush=True)
    xv, rv = View(x, off, pad), View(r, off, pad)
    abi.fused_add_rmsnorm(xv.ptr, wd.data_ptr(), rv.ptr, rows, hidden, xv.stride, rv.stride, DT[dtype], EPS,
                          _stream())
    torch.cuda.synchronize()
    xv.check_outside("input " + tag)
    rv.check_outside("residual " + tag)
    assert_residual_exact(bits(rv.view), o_res, dtype, "fused residual " + tag)
    assert_output_close(bits(xv.view), o_out, dtype, "fused output " + tag)
    del xv, rv

    xa, ov = View(x, off, pad), View(torch.zeros_like(x), off, pad)
    abi.rmsnorm(ov.ptr, xa.ptr, wd.data_ptr(), rows, hidden, ov.stride, xa.stride, DT[dtype], EPS, _stream())
    torch.cuda.synchronize()
    ov.check_outside("plain output " + tag)
    assert_output_close(bits(ov.view), oracle.rmsnorm(bits(x), bits(w), EPS, DT[dtype], threads=th), dtype,
                        "plain " + tag)
    del ov

    ra = View(r, off, pad)
    ov, rov = View(torch.zeros_like(x), off, pad), View(torch.zeros_like(x), off, pad)
    abi.fused_add_rmsnorm_out(ov.ptr, rov.ptr, xa.ptr, ra.ptr, wd.data_ptr(), rows, hidden, ov.stride, rov.stride,
                              xa.stride, ra.stride, DT[dtype], EPS, _stream())
    torch.cuda.synchronize()
    ov.check_outside("out " + tag)
    rov.check_outside("residual_out " + tag)
    assert_residual_exact(bits(rov.view), o_res, dtype, "out residual " + tag)
    assert_output_close(bits(ov.view), o_out, dtype, "out output " + tag)
    del xa, ra, ov, rov

    half = (x.float() / 2).to(dtype)
    parts = [View(half, off, pad), View(half, off, pad)]
    rv, ov = View(r, off, pad), View(torch.zeros_like(x), off, pad)
    abi.reduce_add_rmsnorm(ov.ptr, [p.ptr for p in parts], wd.data_ptr(), rv.ptr, rows, hidden, ov.stride,
                           parts[0].stride, rv.stride, DT[dtype], EPS, _stream())
    torch.cuda.synchronize()
    ov.check_outside("reduce output " + tag)
    rv.check_outside("reduce residual " + tag)
    p_out, p_res = oracle.reduce_add_rmsnorm([bits(half), bits(half)], bits(w), bits(r), EPS, DT[dtype],
                                             threads=th)
    assert_residual_exact(bits(rv.view), p_res, dtype, "reduce residual " + tag)
    assert_output_close(bits(ov.view), p_out, dtype, "reduce output " + tag)


# (hidden, element offset, row padding, dtype): odd widths (every tail length, the
# weight's partial last vector staged) and shifted rows on each staged shape
WLDS_CASES = [(4105, 0, 0, torch.bfloat16), (8191, 0, 0, torch.float16), (8192, 1, 8, torch.bfloat16),
              (12289, 0, 0, torch.bfloat16), (12288, 3, 5, torch.float16), (12294, 0, 0, torch.bfloat16),
              (16383, 0, 0, torch.float16), (16391, 0, 0, torch.bfloat16), (16384, 5, 11, torch.bfloat16),
              (20479, 0, 0, torch.bfloat16), (20483, 0, 0, torch.float16)]


@pytest.mark.parametrize("hidden,off,pad,dtype", WLDS_CASES)
def test_tail_weight_staged_in_lds(abi, hidden, off, pad, dtype):
    """From 1024 rows (plain RMSNorm: 384) the tail variants of 512 x 2-4 and
    1024 x 2-3 load the whole weight into LDS once per workgroup (flags bit
    14) and read each row's shifted vectors from there: modes 0, 1, 3 and 4
    at 1024 rows against the oracle, nothing written outside the views, and
    the dispatch's choice for the odd widths carrying the bit where the
    table stages the weight."""
    rows = 1024
    th = min(16, oracle.max_threads())
    x, r, w = make_inputs(rows, hidden, dtype, seed=hidden + 3 * off)
    o_out, o_res = oracle_fused(x, r, w, EPS, dtype)
    wd = w.to(DEV)
    tag = f"{rows}x{hidden} off {off} pad {pad} {dtype}"
    print("weight staged in LDS", tag, flush=True)
    if hidden % 8:
        # the fused op's staged shapes end with 1024 x 2 (16K), the partial sums' are
        # 512 x 3 (8K-12K), plain RMSNorm's start with 512 x 2 (from 641 vectors)
        staged = {m: bool(abi.select_config(rows, hidden, DT[dtype], m).flags & 16384) for m in (0, 1, 3, 4)}
        assert staged[0] == staged[3] == (hidden < 16384 + 8), staged
        assert staged[4] == (8 * 1025 <= hidden < 8 * 1537), staged
        assert staged[1] == (hidden >= 8 * 641), staged

    xv, rv = View(x, off, pad), View(r, off, pad)
    abi.fused_add_rmsnorm(xv.ptr, wd.data_ptr(), rv.ptr, rows, hidden, xv.stride, rv.stride, DT[dtype], EPS,
                          _stream())
    torch.cuda.synchronize()
    xv.check_outside("input " + tag)
    rv.check_outside("residual " + tag)
    assert_residual_exact(bits(rv.view), o_res, dtype, "fused residual " + tag)
    assert_output_close(bits(xv.view), o_out, dtype, "fused output " + tag)
    del xv, rv

    xa, ov = View(x, off, pad), View(torch.zeros_like(x), off, pad)
    abi.rmsnorm(ov.ptr, xa.ptr, wd.data_ptr(), rows, hidden, ov.stride, xa.stride, DT[dtype], EPS, _stream())
    torch.cuda.synchronize()
    ov.check_outside("plain output " + tag)
    assert_output_close(bits(ov.view), oracle.rmsnorm(bits(x), bits(w), EPS, DT[dtype], threads=th), dtype,
                        "plain " + tag)
    del ov

    ra = View(r, off, pad)
    ov, rov = View(torch.zeros_like(x), off, pad), View(torch.zeros_like(x), off, pad)
    abi.fused_add_rmsnorm_out(ov.ptr, rov.ptr, xa.ptr, ra.ptr, wd.data_ptr(), rows, hidden, ov.stride, rov.stride,
                              xa.stride, ra.stride, DT[dtype], EPS, _stream())
    torch.cuda.synchronize()
    ov.check_outside("out " + tag)
    rov.check_outside("residual_out " + tag)
    assert_residual_exact(bits(rov.view), o_res, dtype, "out residual " + tag)
    assert_output_close(bits(ov.view), o_out, dtype, "out output " + tag)
    del xa, ra, ov, rov

    half = (x.float() / 2).to(dtype)
    parts = [View(half, off, pad), View(half, off, pad)]
    rv, ov = View(r, off, pad), View(torch.zeros_like(x), off, pad)
    abi.reduce_add_rmsnorm(ov.ptr, [p.ptr for p in parts], wd.data_ptr(), rv.ptr, rows, hidden, ov.stride,
                           parts[0].stride, rv.stride, DT[dtype], EPS, _stream())
    torch.cuda.synchronize()
    ov.check_outside("reduce output " + tag)
    rv.check_outside("reduce residual " + tag)
    p_out, p_res = oracle.reduce_add_rmsnorm([bits(half), bits(half)], bits(w), bits(r), EPS, DT[dtype],
                                             threads=th)
    assert_residual_exact(bits(rv.view), p_res, dtype, "reduce residual " + tag)
    assert_output_close(bits(ov.view), p_out, dtype, "reduce output " + tag)


@pytest.mark.parametrize("hidden,off,pad,rows", [(8192, 8, 8, 300), (16384, 1, 8, 300), (4097, 0, 0, 300),
                                                 (16384, 1, 8, 1024)])
def test_off_grid_rows_in_a_hip_graph(abi, hidden, off, pad, rows):
    """Rotated (16-byte aligned off the grid), shifted (2 bytes off) and odd-width rows captured
    in a HIP graph (at 1024 rows the shifted rows' weight staged in LDS): each replay, with fresh
    inputs copied in and eager work between replays, gives the same bits as the eager call on the
    same layout."""
    import hp_rms_norm_amd
    dtype, eps = torch.bfloat16, 1e-6
    stride = hidden + off + pad
    bx = torch.zeros(rows, stride, dtype=dtype, device=DEV)
    br = torch.zeros_like(bx)
    xs, rs = bx[:, off:off + hidden], br[:, off:off + hidden]
    wd = make_inputs(1, hidden, dtype, 0)[2].to(DEV)
    print("off-grid graph", hidden, off, pad, rows, flush=True)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        hp_rms_norm_amd.hp_rms_norm(xs, wd, rs, eps)  # warm-up outside the graph
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        hp_rms_norm_amd.hp_rms_norm(xs, wd, rs, eps)
    ex, er = torch.zeros_like(bx), torch.zeros_like(br)
    xe, re_ = ex[:, off:off + hidden], er[:, off:off + hidden]
    for rep in range(4):
        x, r, _ = make_inputs(rows, hidden, dtype, 200 + rep)
        xs.copy_(x.to(DEV))
        rs.copy_(r.to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        got_x, got_r = u16(xs), u16(rs)
        xe.copy_(x.to(DEV))
        re_.copy_(r.to(DEV))
        hp_rms_norm_amd.hp_rms_norm(xe, wd, re_, eps)
        torch.cuda.synchronize()
        assert torch.equal(got_x, u16(xe)), f"replay {rep} output"
        assert torch.equal(got_r, u16(re_)), f"replay {rep} residual"
    o_out, o_res = oracle_fused(x, r, wd.cpu(), eps, dtype)
    assert_residual_exact(got_r.numpy().view(np.uint16), o_res, dtype, "graph residual")
    assert_output_close(got_x.numpy().view(np.uint16), o_out, dtype, "graph output")


# ---- modes 1-4 -------------------------------------------------------------------------
OTHER_WIDTHS = [8, 1000, 1001, 4096, 4103, 12288, 16384, 16391, 32768, 32775, 65536]


@pytest.mark.parametrize("hidden", OTHER_WIDTHS)
def test_plain_fp8_out_and_reduce_on_misaligned_rows(abi, hidden):
    dtype, rows = torch.float16, 37
    x, r, w = make_inputs(rows, hidden, dtype, seed=hidden)
    print("modes 1-4 misaligned", hidden, flush=True)
    wv = View(w[None], 1, 0)
    tag = f"{rows}x{hidden}"

    # plain RMSNorm: input at a 2-byte offset, output 16-byte aligned off the 128-byte grid
    xv, ov = View(x, 1, 4), View(torch.zeros_like(x), 8, 3)
    abi.rmsnorm(ov.ptr, xv.ptr, wv.ptr, rows, hidden, ov.stride, xv.stride, DT[dtype], EPS, _stream())
    xa, oa = x.to(DEV), torch.empty(rows, hidden, dtype=dtype, device=DEV)
    abi.rmsnorm(oa.data_ptr(), xa.data_ptr(), w.to(DEV).data_ptr(), rows, hidden, hidden, hidden, DT[dtype], EPS,
                _stream())
    torch.cuda.synchronize()
    ov.check_outside("plain output")
    want = oracle.rmsnorm(bits(x), bits(w), EPS, DT[dtype], threads=min(16, oracle.max_threads()))
    assert_output_close(bits(ov.view), want, dtype, "plain " + tag)

    # FP8 output at an odd byte offset
    xv, rv = View(x, 1, 2), View(r, 3, 0)
    qv = ByteView(rows, hidden, 3, 5)
    sc = torch.empty(rows, dtype=torch.float32, device=DEV)
    abi.fused_add_rmsnorm_fp8(qv.ptr, sc.data_ptr(), xv.ptr, wv.ptr, rv.ptr, rows, hidden, qv.stride, xv.stride,
                              rv.stride, DT[dtype], EPS, _stream())
    torch.cuda.synchronize()
    qv.check_outside("fp8 output")
    xv.check_outside("fp8 input")
    assert torch.equal(u16(xv.view), u16(x)), "fp8: input modified " + tag
    oq, osc, ores = oracle.fused_add_rmsnorm_fp8(bits(x), bits(w), bits(r), EPS, DT[dtype],
                                                 threads=min(16, oracle.max_threads()))
    assert_residual_exact(bits(rv.view), ores, dtype, "fp8 residual " + tag)
    assert oracle.e4m3_ulp_distance(qv.view.contiguous().cpu().numpy(), oq).max() <= 1, "fp8 " + tag
    np.testing.assert_allclose(sc.cpu().numpy(), osc, rtol=2.0 ** -7)

    # out of place: every stream at its own offset
    xv, rv = View(x, 1, 2), View(r, 2, 1)
    ov, rov = View(torch.zeros_like(x), 3, 0), View(torch.zeros_like(x), 5, 2)
    abi.fused_add_rmsnorm_out(ov.ptr, rov.ptr, xv.ptr, rv.ptr, wv.ptr, rows, hidden, ov.stride, rov.stride,
                              xv.stride, rv.stride, DT[dtype], EPS, _stream())
    torch.cuda.synchronize()
    ov.check_outside("out")
    rov.check_outside("residual_out")
    assert torch.equal(u16(xv.view), u16(x)) and torch.equal(u16(rv.view), u16(r)), "out: inputs modified " + tag
    o_out, o_res = oracle_fused(x, r, w, EPS, dtype)
    assert_residual_exact(bits(rov.view), o_res, dtype, "out residual " + tag)
    assert_output_close(bits(ov.view), o_out, dtype, "out output " + tag)

    # partial sums: three parts sharing one row stride at different offsets
    g = torch.Generator().manual_seed(hidden)
    parts = [torch.randn((rows, hidden), generator=g).to(dtype) for _ in range(3)]
    stride = hidden + 7
    pbuf = torch.zeros(3, rows, stride + 4, dtype=dtype, device=DEV)
    pviews = [pbuf[i, :, 1 + i:1 + i + hidden] for i in range(3)]
    for pvw, p in zip(pviews, parts):
        pvw.copy_(p.to(DEV))
    rv, ov = View(r, 1, 0), View(torch.zeros_like(x), 2, 1)
    abi.reduce_add_rmsnorm(ov.ptr, [p.data_ptr() for p in pviews], wv.ptr, rv.ptr, rows, hidden, ov.stride,
                           pbuf.shape[2], rv.stride, DT[dtype], EPS, _stream())
    torch.cuda.synchronize()
    ov.check_outside("reduce output")
    o_out, o_res = oracle.reduce_add_rmsnorm([bits(p) for p in parts], bits(w), bits(r), EPS, DT[dtype],
                                             threads=min(16, oracle.max_threads()))
    assert_residual_exact(bits(rv.view), o_res, dtype, "reduce residual " + tag)
    assert_output_close(bits(ov.view), o_out, dtype, "reduce output " + tag)


# ---- shifted rows: the written streams share one phase ----------------------------------
SHIFT_WIDTHS = [4104, 4105, 8195, 16384, 32773]


@pytest.mark.parametrize("hidden", SHIFT_WIDTHS)
@pytest.mark.parametrize("dtype,rows,nparts", [(torch.bfloat16, 21, 3), (torch.float16, 300, 8),
                                               (torch.float16, 64, 8)],
                         ids=["bf16-latency-table", "fp16-bandwidth-table", "fp16-latency-table-8-parts"])
def test_shifted_rows_every_mode(abi, hidden, dtype, rows, nparts):
    """From 513 whole vectors up, rows of calls whose streams are all off
    16-byte alignment (element offsets 1-7; row strides not a multiple of 8,
    so each row has its own shift) are shifted to the first written stream's
    phase: modes 0-4 against the oracle, with the written streams at one phase
    and the read streams at others (the FP8 output: every stream at one
    phase), and nothing written outside the views; on the latency table's
    shapes (few rows) and the bandwidth table's."""
    x, r, w = make_inputs(rows, hidden, dtype, seed=hidden + 7)
    tag = f"{rows}x{hidden} {dtype}"
    print("shifted rows", tag, flush=True)
    th = min(16, oracle.max_threads())
    o_out, o_res = oracle_fused(x, r, w, EPS, dtype)
    wv = View(w[None], 1, 0)

    # the fused op: input and residual at one phase
    xv, rv = View(x, 3, 2), View(r, 3, 2)
    abi.fused_add_rmsnorm(xv.ptr, wv.ptr, rv.ptr, rows, hidden, xv.stride, rv.stride, DT[dtype], EPS, _stream())
    torch.cuda.synchronize()
    xv.check_outside("input")
    rv.check_outside("residual")
    assert_residual_exact(bits(rv.view), o_res, dtype, "fused residual " + tag)
    assert_output_close(bits(xv.view), o_out, dtype, "fused output " + tag)

    # plain RMSNorm: the output decides
    xv, ov = View(x, 2, 1), View(torch.zeros_like(x), 5, 3)
    abi.rmsnorm(ov.ptr, xv.ptr, wv.ptr, rows, hidden, ov.stride, xv.stride, DT[dtype], EPS, _stream())
    torch.cuda.synchronize()
    ov.check_outside("plain output")
    want = oracle.rmsnorm(bits(x), bits(w), EPS, DT[dtype], threads=th)
    assert_output_close(bits(ov.view), want, dtype, "plain " + tag)

    # FP8 output: the input's and the residual's element phase equals the byte rows' phase
    xv, rv, qv = View(x, 1, 2), View(r, 1, 2), ByteView(rows, hidden, 1, 2)
    sc = torch.empty(rows, dtype=torch.float32, device=DEV)
    abi.fused_add_rmsnorm_fp8(qv.ptr, sc.data_ptr(), xv.ptr, wv.ptr, rv.ptr, rows, hidden, qv.stride, xv.stride,
                              rv.stride, DT[dtype], EPS, _stream())
    torch.cuda.synchronize()
    qv.check_outside("fp8 output")
    rv.check_outside("fp8 residual")
    oq, osc, ores = oracle.fused_add_rmsnorm_fp8(bits(x), bits(w), bits(r), EPS, DT[dtype], threads=th)
    assert_residual_exact(bits(rv.view), ores, dtype, "fp8 residual " + tag)
    assert oracle.e4m3_ulp_distance(qv.view.contiguous().cpu().numpy(), oq).max() <= 1, "fp8 " + tag
    np.testing.assert_allclose(sc.cpu().numpy(), osc, rtol=2.0 ** -7)

    # out of place: both outputs at one phase
    xv, rv = View(x, 2, 3), View(r, 2, 0)
    ov, rov = View(torch.zeros_like(x), 7, 1), View(torch.zeros_like(x), 7, 1)
    abi.fused_add_rmsnorm_out(ov.ptr, rov.ptr, xv.ptr, rv.ptr, wv.ptr, rows, hidden, ov.stride, rov.stride,
                              xv.stride, rv.stride, DT[dtype], EPS, _stream())
    torch.cuda.synchronize()
    ov.check_outside("out")
    rov.check_outside("residual_out")
    assert_residual_exact(bits(rov.view), o_res, dtype, "out residual " + tag)
    assert_output_close(bits(ov.view), o_out, dtype, "out output " + tag)

    # partial sums: the output and the residual at one phase, the parts elsewhere
    g = torch.Generator().manual_seed(hidden)
    parts = [torch.randn((rows, hidden), generator=g).to(dtype) for _ in range(nparts)]
    pbuf = torch.zeros(nparts, rows, hidden + 11, dtype=dtype, device=DEV)
    pviews = [pbuf[i, :, 1 + i % 7:1 + i % 7 + hidden] for i in range(nparts)]
    for pvw, p in zip(pviews, parts):
        pvw.copy_(p.to(DEV))
    rv, ov = View(r, 4, 6), View(torch.zeros_like(x), 4, 6)
    abi.reduce_add_rmsnorm(ov.ptr, [p.data_ptr() for p in pviews], wv.ptr, rv.ptr, rows, hidden, ov.stride,
                           pbuf.shape[2], rv.stride, DT[dtype], EPS, _stream())
    torch.cuda.synchronize()
    ov.check_outside("reduce output")
    rv.check_outside("reduce residual")
    o_out, o_res = oracle.reduce_add_rmsnorm([bits(p) for p in parts], bits(w), bits(r), EPS, DT[dtype], threads=th)
    assert_residual_exact(bits(rv.view), o_res, dtype, "reduce residual " + tag)
    assert_output_close(bits(ov.view), o_out, dtype, "reduce output " + tag)


# ---- modes 5, 6: the MX outputs --------------------------------------------------------
@pytest.mark.parametrize("fmt", ["mxfp8", "mxfp4"])
def test_mx_on_misaligned_rows_equals_the_aligned_kernel(abi, fmt):
    """Input and residual at 2-byte offsets, the elements and the scales at odd
    byte offsets: the same bytes as the aligned call, nothing written outside."""
    f = abi.MX_FP8_E4M3 if fmt == "mxfp8" else abi.MX_FP4_E2M1
    dtype = torch.bfloat16
    for hidden in (256, 2048, 4096, 16384, 32768):
        for rows in (67, 3):
            x, r, w = make_inputs(rows, hidden, dtype, seed=hidden + rows)
            qw = hidden if fmt == "mxfp8" else hidden // 2
            print("mx misaligned", fmt, rows, hidden, flush=True)
            # aligned reference call
            xa, ra, wa = x.to(DEV), r.to(DEV), w.to(DEV)
            qa = torch.empty(rows, qw, dtype=torch.uint8, device=DEV)
            sa = torch.empty(rows, hidden // 32, dtype=torch.uint8, device=DEV)
            abi.fused_add_rmsnorm_mx(qa.data_ptr(), sa.data_ptr(), xa.data_ptr(), wa.data_ptr(), ra.data_ptr(), rows,
                                     hidden, qw, hidden // 32, hidden, hidden, f, DT[dtype], EPS, _stream())
            xv, rv, wv = View(x, 1, 2), View(r, 5, 0), View(w[None], 1, 0)
            qv, sv = ByteView(rows, qw, 3, 2), ByteView(rows, hidden // 32, 1, 3)
            abi.fused_add_rmsnorm_mx(qv.ptr, sv.ptr, xv.ptr, wv.ptr, rv.ptr, rows, hidden, qv.stride, sv.stride,
                                     xv.stride, rv.stride, f, DT[dtype], EPS, _stream())
            torch.cuda.synchronize()
            tag = f"{fmt} {rows}x{hidden}"
            qv.check_outside("mx elements " + tag)
            sv.check_outside("mx scales " + tag)
            xv.check_outside("mx input " + tag)
            rv.check_outside("mx residual " + tag)
            assert torch.equal(u16(rv.view), u16(ra)), "residual " + tag
            assert torch.equal(sv.view.cpu(), sa.cpu()), "scales " + tag
            assert torch.equal(qv.view.cpu(), qa.cpu()), "elements " + tag
            assert torch.equal(u16(xv.view), u16(x)), "input modified " + tag


# ---- the general tier in every mode -------------------------------------------------------
def strided_rows(t, stride):
    """A [rows, hidden] device view with the given row stride over a flat buffer
    of (rows - 1) * stride + hidden elements (no storage between the rows)."""
    rows, hidden = t.shape
    flat = torch.zeros((rows - 1) * stride + hidden, dtype=t.dtype, device=DEV)
    v = flat.as_strided((rows, hidden), (stride, 1))
    v.copy_(t.to(DEV))
    return v


# hidden < 8 (the general register kernel), > 65543 (the two-pass kernel), and 101 with a
# row stride of 2^27 elements: its table shape puts 16 rows in a workgroup, whose buffer
# resources would span 4 GiB, so the vector shapes are refused and the register kernel takes
# the call.  1001 with a stride of 2^28 stays on the vector tier: with 2 rows the latency
# table gives one row per workgroup, so huge strides fit its resources.  The vector kernels
# take 32-bit row strides: 4096 with 2^31 - 8 (the largest, rows 16 bytes off the grid) stays
# on the vector tier, 1001 with 2^31 goes to the register kernel (4 GiB buffers).
GENERAL_CASES = [(7, 5, 7), (70001, 3, 70001), (101, 2, 1 << 27), (1001, 2, 1 << 28), (4096, 2, (1 << 31) - 8),
                 (1001, 2, 1 << 31)]


@pytest.mark.parametrize("hidden,rows,stride", GENERAL_CASES)
def test_general_tier_every_mode(abi, hidden, rows, stride):
    dtype = torch.bfloat16
    x, r, w = make_inputs(rows, hidden, dtype, seed=hidden)
    wd = w.to(DEV)
    tag = f"{rows}x{hidden} stride {stride}"
    print("general tier", tag, flush=True)
    threads = min(16, oracle.max_threads())
    o_out, o_res = oracle_fused(x, r, w, EPS, dtype)

    # mode 0, in place
    xd, rd = strided_rows(x, stride), strided_rows(r, stride)
    abi.fused_add_rmsnorm(xd.data_ptr(), wd.data_ptr(), rd.data_ptr(), rows, hidden, stride, stride, DT[dtype], EPS,
                          _stream())
    torch.cuda.synchronize()
    assert_residual_exact(bits(rd), o_res, dtype, "fused residual " + tag)
    assert_output_close(bits(xd), o_out, dtype, "fused output " + tag)
    del xd, rd

    # mode 1, plain RMSNorm
    xd, od = strided_rows(x, stride), strided_rows(torch.zeros_like(x), stride)
    abi.rmsnorm(od.data_ptr(), xd.data_ptr(), wd.data_ptr(), rows, hidden, stride, stride, DT[dtype], EPS, _stream())
    torch.cuda.synchronize()
    assert_output_close(bits(od), oracle.rmsnorm(bits(x), bits(w), EPS, DT[dtype], threads=threads), dtype,
                        "plain " + tag)
    del xd, od

    # mode 2, FP8 output (rows of `stride` bytes)
    xd, rd = strided_rows(x, stride), strided_rows(r, stride)
    qflat = torch.zeros((rows - 1) * stride + hidden, dtype=torch.uint8, device=DEV)
    q = qflat.as_strided((rows, hidden), (stride, 1))
    sc = torch.empty(rows, dtype=torch.float32, device=DEV)
    abi.fused_add_rmsnorm_fp8(q.data_ptr(), sc.data_ptr(), xd.data_ptr(), wd.data_ptr(), rd.data_ptr(), rows, hidden,
                              stride, stride, stride, DT[dtype], EPS, _stream())
    torch.cuda.synchronize()
    oq, osc, ores = oracle.fused_add_rmsnorm_fp8(bits(x), bits(w), bits(r), EPS, DT[dtype], threads=threads)
    assert_residual_exact(bits(rd), ores, dtype, "fp8 residual " + tag)
    assert oracle.e4m3_ulp_distance(q.contiguous().cpu().numpy(), oq).max() <= 1, "fp8 " + tag
    np.testing.assert_allclose(sc.cpu().numpy(), osc, rtol=2.0 ** -7)
    del xd, rd, qflat, q

    # mode 3, out of place
    xd, rd = strided_rows(x, stride), strided_rows(r, stride)
    od, rod = strided_rows(torch.zeros_like(x), stride), strided_rows(torch.zeros_like(x), stride)
    abi.fused_add_rmsnorm_out(od.data_ptr(), rod.data_ptr(), xd.data_ptr(), rd.data_ptr(), wd.data_ptr(), rows,
                              hidden, stride, stride, stride, stride, DT[dtype], EPS, _stream())
    torch.cuda.synchronize()
    assert_residual_exact(bits(rod), o_res, dtype, "out residual " + tag)
    assert_output_close(bits(od), o_out, dtype, "out output " + tag)
    del xd, rd, od, rod

    # mode 4, three partial sums
    g = torch.Generator().manual_seed(hidden + 1)
    parts = [torch.randn((rows, hidden), generator=g).to(dtype) for _ in range(3)]
    pds = [strided_rows(p, stride) for p in parts]
    rd, od = strided_rows(r, stride), strided_rows(torch.zeros_like(x), stride)
    abi.reduce_add_rmsnorm(od.data_ptr(), [p.data_ptr() for p in pds], wd.data_ptr(), rd.data_ptr(), rows, hidden,
                           stride, stride, stride, DT[dtype], EPS, _stream())
    torch.cuda.synchronize()
    p_out, p_res = oracle.reduce_add_rmsnorm([bits(p) for p in parts], bits(w), bits(r), EPS, DT[dtype],
                                             threads=threads)
    assert_residual_exact(bits(rd), p_res, dtype, "reduce residual " + tag)
    assert_output_close(bits(od), p_out, dtype, "reduce output " + tag)
