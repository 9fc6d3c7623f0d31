"""ctypes wrapper of the CPU oracle ``oracle/libhprms_oracle.so``.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``, as the checker or the timed CPU
baseline.  The product package ``hp_rms_norm_amd`` never imports it.

Arrays are numpy ``uint16`` holding bfloat16 / binary16 bit patterns, 2-D
``[rows, hidden]`` with contiguous rows (any row stride).  The arithmetic and
the reference lines it restates are documented in ``oracle/hprms_oracle.c``.
"""
import ctypes
import os

import numpy as np

BF16, FP16 = 0, 1
COPY, RELU = 0, 1

# planted mistakes understood by the C oracle (tests/test_oracle.py shows that
# the pins reject each of them)
MUTATIONS = {
    "drop_eps": 1,
    "mean_h_minus_1": 2,
    "weight_reversed": 3,
    "trunc_residual": 4,
    "norm_input": 5,
    "l1_mean": 6,
    "unrounded_squares": 7,
    "weight_twice": 8,
    "binary64_squares": 9,
}

# planted mistakes of the partial-sum step (reduce_add_rmsnorm)
REDUCE_MUTATIONS = {
    "step_rounding": 1,
    "no_rounding": 2,
    "reversed": 3,
}

# planted mistakes of the MX quantisation step (fused_add_rmsnorm_mx)
MX_MUTATIONS = {
    "ceil_scale": 1,
    "emax_plus_1": 2,
    "truncate": 3,
    "nibbles_swapped": 4,
}
MXFP8, MXFP4 = 0, 1

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libhprms_oracle.so")
_lib = None

_u16p = ctypes.POINTER(ctypes.c_uint16)
_f32p = ctypes.POINTER(ctypes.c_float)
_i64 = ctypes.c_int64


def build():
    """Compile the oracle with its Makefile (gcc, OpenMP)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run `make -C oracle` (or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        L.hprms_oracle_fused_add_rmsnorm.argtypes = [_u16p, _u16p, _u16p, _i64, _i64, _i64, _i64,
                                                     ctypes.c_int, ctypes.c_double, ctypes.c_int, ctypes.c_int]
        L.hprms_oracle_rmsnorm.argtypes = [_u16p, _u16p, _u16p, _i64, _i64, _i64, _i64,
                                           ctypes.c_int, ctypes.c_double, ctypes.c_int]
        L.hprms_oracle_streamer.argtypes = [_u16p, _u16p, _i64, _i64, _i64, _i64,
                                            ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.hprms_oracle_from_f32.argtypes = [_f32p, _u16p, _i64, ctypes.c_int]
        L.hprms_oracle_to_f32.argtypes = [_u16p, _f32p, _i64, ctypes.c_int]
        L.hprms_oracle_max_threads.restype = ctypes.c_int
        _u8p = ctypes.POINTER(ctypes.c_uint8)
        L.hprms_oracle_fused_add_rmsnorm_fp8.argtypes = [_u8p, _f32p, _u16p, _u16p, _u16p, _i64, _i64, _i64,
                                                         _i64, _i64, ctypes.c_int, ctypes.c_double, ctypes.c_int]
        L.hprms_oracle_e4m3_from_f32.argtypes = [_f32p, _u8p, _i64]
        L.hprms_oracle_fused_add_rmsnorm_mx.argtypes = [_u8p, _u8p, _u16p, _u16p, _u16p, _i64, _i64, _i64, _i64,
                                                        _i64, _i64, ctypes.c_int, ctypes.c_int, ctypes.c_double,
                                                        ctypes.c_int, ctypes.c_int]
        L.hprms_oracle_e2m1_from_f32.argtypes = [_f32p, _u8p, _i64]
        L.hprms_oracle_mx_quantize.argtypes = [_u8p, _u8p, _u16p, _i64, _i64, ctypes.c_int, ctypes.c_int,
                                               ctypes.c_int]
        L.hprms_oracle_reduce_add_rmsnorm.argtypes = [_u16p, ctypes.POINTER(_u16p), ctypes.c_int, _u16p, _u16p,
                                                      _i64, _i64, _i64, _i64, _i64, ctypes.c_int,
                                                      ctypes.c_double, ctypes.c_int, ctypes.c_int]
        _lib = L
    return _lib


def _p16(a):
    return a.ctypes.data_as(_u16p)


def _rows(a):
    assert a.dtype == np.uint16 and a.ndim == 2 and a.strides[1] == 2, "2-D uint16 rows expected"
    assert a.strides[0] % 2 == 0
    return a.shape[0], a.shape[1], a.strides[0] // 2


def max_threads():
    return lib().hprms_oracle_max_threads()


def fused_add_rmsnorm_(x, w, r, eps, dtype, threads=1, mutation=0):
    """In place, like the op: r <- rne(x + r); x <- normalised output."""
    rows, hidden, sx = _rows(x)
    rows_r, hidden_r, sr = _rows(r)
    assert (rows, hidden) == (rows_r, hidden_r) and w.shape == (hidden,) and w.dtype == np.uint16
    w = np.ascontiguousarray(w)
    if isinstance(mutation, str):
        mutation = MUTATIONS[mutation]
    rc = lib().hprms_oracle_fused_add_rmsnorm(_p16(x), _p16(w), _p16(r), rows, hidden, max(sx, hidden),
                                              max(sr, hidden), dtype, float(eps), threads, mutation)
    if rc != 0:
        raise ValueError(f"oracle rejected the arguments ({rc})")


def fused_add_rmsnorm(x, w, r, eps, dtype, threads=1, mutation=0):
    """Out of place: returns (output, new_residual) as fresh arrays."""
    xo = np.array(x, dtype=np.uint16, copy=True, order="C")
    ro = np.array(r, dtype=np.uint16, copy=True, order="C")
    fused_add_rmsnorm_(xo, w, ro, eps, dtype, threads, mutation)
    return xo, ro


def rmsnorm(x, w, eps, dtype, threads=1):
    xc = np.ascontiguousarray(x)
    rows, hidden, sx = _rows(xc)
    out = np.empty_like(xc)
    rc = lib().hprms_oracle_rmsnorm(_p16(out), _p16(xc), _p16(np.ascontiguousarray(w)), rows, hidden,
                                    hidden, sx, dtype, float(eps), threads)
    if rc != 0:
        raise ValueError(f"oracle rejected the arguments ({rc})")
    return out


def streamer(x, dtype, op, threads=1):
    xc = np.ascontiguousarray(x)
    rows, hidden, sx = _rows(xc)
    out = np.empty_like(xc)
    rc = lib().hprms_oracle_streamer(_p16(out), _p16(xc), rows, hidden, hidden, sx, dtype, op, threads)
    if rc != 0:
        raise ValueError(f"oracle rejected the arguments ({rc})")
    return out


def reduce_add_rmsnorm(parts, w, r, eps, dtype, threads=1, mutation=0):
    """Partial-sum form: a = rne(sum of ``parts`` in order, fp32), then the
    fused op on a.  Returns (output, new_residual) as fresh arrays; the
    arguments are not modified."""
    ps = [np.ascontiguousarray(p, dtype=np.uint16) for p in parts]
    assert ps and all(p.shape == ps[0].shape for p in ps)
    rows, hidden, _ = _rows(ps[0])
    ro = np.array(r, dtype=np.uint16, copy=True, order="C")
    assert ro.shape == (rows, hidden)
    out = np.empty((rows, hidden), dtype=np.uint16)
    if isinstance(mutation, str):
        mutation = REDUCE_MUTATIONS[mutation]
    arr = (_u16p * len(ps))(*[_p16(p) for p in ps])
    rc = lib().hprms_oracle_reduce_add_rmsnorm(_p16(out), arr, len(ps), _p16(np.ascontiguousarray(w)), _p16(ro),
                                               rows, hidden, hidden, hidden, hidden, dtype, float(eps), threads,
                                               mutation)
    if rc != 0:
        raise ValueError(f"oracle rejected the arguments ({rc})")
    return out, ro


def from_f32(a, dtype):
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().hprms_oracle_from_f32(a.ctypes.data_as(_f32p), _p16(out), a.size, dtype)
    return out


def to_f32(a, dtype):
    a = np.ascontiguousarray(a, dtype=np.uint16)
    out = np.empty(a.shape, dtype=np.float32)
    lib().hprms_oracle_to_f32(_p16(a), out.ctypes.data_as(_f32p), a.size, dtype)
    return out


def ulp_distance(a, b, dtype):
    """Distance in units of the last place between two arrays of 16-bit
    patterns (bf16 or fp16), on the ordered-integer line; NaN pairs count 0,
    NaN against a number counts as a large distance."""
    a = np.asarray(a, dtype=np.uint16).astype(np.int32)
    b = np.asarray(b, dtype=np.uint16).astype(np.int32)

    def ordered(v):
        mag = v & 0x7FFF
        return np.where(v & 0x8000, -mag, mag)

    nan_floor = 0x7F80 if dtype == BF16 else 0x7C00
    na = (a & 0x7FFF) > nan_floor
    nb = (b & 0x7FFF) > nan_floor
    d = np.abs(ordered(a) - ordered(b))
    d = np.where(na & nb, 0, d)
    d = np.where(na ^ nb, 1 << 20, d)
    return d


def fused_add_rmsnorm_fp8(x, w, r, eps, dtype, threads=1):
    """FP8 form: returns (q uint8 [rows, hidden] of e4m3fn bits, scale float32
    [rows], new residual); x is not modified."""
    xc = np.ascontiguousarray(x)
    rows, hidden, sx = _rows(xc)
    ro = np.array(r, dtype=np.uint16, copy=True, order="C")
    q = np.empty((rows, hidden), dtype=np.uint8)
    sc = np.empty(rows, dtype=np.float32)
    rc = lib().hprms_oracle_fused_add_rmsnorm_fp8(
        q.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), sc.ctypes.data_as(_f32p), _p16(xc),
        _p16(np.ascontiguousarray(w)), _p16(ro), rows, hidden, hidden, sx, hidden, dtype, float(eps), threads)
    if rc != 0:
        raise ValueError(f"oracle rejected the arguments ({rc})")
    return q, sc, ro


def fused_add_rmsnorm_fp8_ub(x, w, r, eps, dtype, scale_ub, threads=1, bound_scale=False):
    """FP8 form with per-row scales whose row maximum is bounded above (the
    activation scale bound of FP8 row-wise checkpoints): returns (q uint8
    [rows, hidden] of e4m3fn bits, scale float32 [rows], new residual).  With
    amax the row's max |y| (NaN if the row holds a NaN), amax' = scale_ub
    where amax > scale_ub (a NaN bound bounds nothing), scale = max(amax' /
    448, FLT_MIN) and q = e4m3fn(clamp(y * (1 / scale), -448, 448)): the
    quantisation step of hprms_oracle_fused_add_rmsnorm_fp8 with the bounded
    maximum.  `bound_scale` (bounding the scale by scale_ub instead of the
    maximum) exists for the test that plants that mistake."""
    y, res = fused_add_rmsnorm(x, w, r, eps, dtype, threads=threads)
    yf = to_f32(y, dtype)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        amax = np.abs(yf).max(axis=1).astype(np.float32)
        ub = np.float32(scale_ub)
        if not bound_scale:
            amax = np.where(amax > ub, ub, amax).astype(np.float32)
        sc = (amax / np.float32(448.0)).astype(np.float32)
        if bound_scale:
            sc = np.where(sc > ub, ub, sc).astype(np.float32)
        tiny = np.float32(np.finfo(np.float32).tiny)
        sc = np.where(sc < tiny, tiny, sc).astype(np.float32)
        isc = (np.float32(1.0) / sc).astype(np.float32)
        v = (yf * isc[:, None]).astype(np.float32)
        v = np.where(v > 448.0, np.float32(448.0), np.where(v < -448.0, np.float32(-448.0), v)).astype(np.float32)
    return e4m3_from_f32(v), sc, res


def fused_add_rmsnorm_fp8_static(x, w, r, eps, dtype, scale, threads=1):
    """FP8 form with one given scale for every row (static per-tensor
    quantisation): returns (q uint8 [rows, hidden] of e4m3fn bits, new
    residual), q = e4m3fn(clamp(y * (1 / scale), -448, 448)) with y the fused
    op's 16-bit output (fused_add_rmsnorm) and 1 / scale rounded to binary32,
    the dynamic form's quantisation step (hprms_oracle_fused_add_rmsnorm_fp8)
    with the scale given instead of taken from the row maximum."""
    y, res = fused_add_rmsnorm(x, w, r, eps, dtype, threads=threads)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        isc = np.float32(1.0) / np.float32(scale)
        v = to_f32(y, dtype) * isc
        v = np.where(v > 448.0, np.float32(448.0), np.where(v < -448.0, np.float32(-448.0), v)).astype(np.float32)
    return e4m3_from_f32(v), res


def fused_add_rmsnorm_fp8_group(x, w, r, eps, dtype, threads=1, group=128, floor=True):
    """FP8 form with one scale per `group` (128) consecutive elements of a
    row: returns (q uint8 [rows, hidden] of e4m3fn bits, scales float32
    [rows, hidden // group], new residual).  Per group, scale = max(amax|y| /
    448, FLT_MIN) (NaN if the group holds a NaN) and q = e4m3fn(clamp(y * (1 /
    scale), -448, 448)) with y the fused op's 16-bit output: the per-row step
    of hprms_oracle_fused_add_rmsnorm_fp8 applied to each group.  `group` and
    `floor` (the FLT_MIN floor) exist for the tests that plant mistakes."""
    y, res = fused_add_rmsnorm(x, w, r, eps, dtype, threads=threads)
    rows, hidden = y.shape
    if hidden % group:
        raise ValueError(f"hidden {hidden} is not a multiple of the group size {group}")
    yf = to_f32(y, dtype).reshape(rows, hidden // group, group)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        amax = np.max(np.abs(yf), axis=-1)                       # NaN propagates
        sc = (amax / np.float32(448.0)).astype(np.float32)
        if floor:
            tiny = np.float32(np.finfo(np.float32).tiny)
            sc = np.where(sc < tiny, tiny, sc).astype(np.float32)  # NaN compares false and stays
        isc = (np.float32(1.0) / sc).astype(np.float32)
        v = yf * isc[..., None]
        v = np.where(v > 448.0, np.float32(448.0), np.where(v < -448.0, np.float32(-448.0), v)).astype(np.float32)
    return e4m3_from_f32(v).reshape(rows, hidden), sc, res


def e4m3_from_f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint8)
    lib().hprms_oracle_e4m3_from_f32(a.ctypes.data_as(_f32p), out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)),
                                     a.size)
    return out


def e4m3_ulp_distance(a, b):
    """Distance between FP8 e4m3fn bit patterns on the ordered line; NaN pairs 0."""
    a = np.asarray(a, dtype=np.uint8).astype(np.int32)
    b = np.asarray(b, dtype=np.uint8).astype(np.int32)

    def ordered(v):
        mag = v & 0x7F
        return np.where(v & 0x80, -mag, mag)

    na, nb = (a & 0x7F) == 0x7F, (b & 0x7F) == 0x7F
    d = np.abs(ordered(a) - ordered(b))
    d = np.where(na & nb, 0, d)
    return np.where(na ^ nb, 1 << 20, d)


def fused_add_rmsnorm_mx(x, w, r, eps, dtype, elem, threads=1, mutation=0):
    """OCP MX form: returns (q uint8 [rows, H] (MXFP8) or [rows, H/2] (MXFP4,
    two E2M1 codes per byte, the even element in the low nibble), scales uint8
    [rows, H/32] (E8M0), new residual); x is not modified."""
    xc = np.ascontiguousarray(x)
    rows, hidden, sx = _rows(xc)
    ro = np.array(r, dtype=np.uint16, copy=True, order="C")
    qw = hidden if elem == MXFP8 else hidden // 2
    q = np.zeros((rows, qw), dtype=np.uint8)
    sc = np.zeros((rows, max(1, hidden // 32)), dtype=np.uint8)
    if isinstance(mutation, str):
        mutation = MX_MUTATIONS[mutation]
    _u8 = ctypes.POINTER(ctypes.c_uint8)
    rc = lib().hprms_oracle_fused_add_rmsnorm_mx(q.ctypes.data_as(_u8), sc.ctypes.data_as(_u8), _p16(xc),
                                                 _p16(np.ascontiguousarray(w)), _p16(ro), rows, hidden, qw,
                                                 sc.shape[1], sx, hidden, elem, dtype, float(eps), threads, mutation)
    if rc != 0:
        raise ValueError(f"oracle rejected the arguments ({rc})")
    return q, sc, ro


def e2m1_from_f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint8)
    lib().hprms_oracle_e2m1_from_f32(a.ctypes.data_as(_f32p), out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)),
                                     a.size)
    return out


def mx_quantize(y, dtype, elem, mutation=0):
    """The MX step alone on [rows, H] 16-bit patterns: returns (q, scales)."""
    yc = np.ascontiguousarray(y, dtype=np.uint16)
    rows, hidden = yc.shape
    q = np.zeros((rows, hidden if elem == MXFP8 else hidden // 2), dtype=np.uint8)
    sc = np.zeros((rows, hidden // 32), dtype=np.uint8)
    if isinstance(mutation, str):
        mutation = MX_MUTATIONS[mutation]
    _u8 = ctypes.POINTER(ctypes.c_uint8)
    rc = lib().hprms_oracle_mx_quantize(q.ctypes.data_as(_u8), sc.ctypes.data_as(_u8), _p16(yc), rows, hidden, elem,
                                        dtype, mutation)
    if rc != 0:
        raise ValueError(f"oracle rejected the arguments ({rc})")
    return q, sc
