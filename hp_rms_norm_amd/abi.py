"""ctypes binding of the C ABI of ``libhprms.so`` (include/hp_rms_norm_amd.h).

This is the binding a caller without the torch extension would use; the
tests use it to drive the kernels through the C ABI directly.  ``BENCH`` binds
the same ABI in the bench library ``libhprms_bench.so``, which bench.py and
the tuning tests load for the kernel shapes no table row selects.  Device
pointers and streams are plain integers (e.g. ``tensor.data_ptr()`` and
``torch.cuda.current_stream().cuda_stream``).
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
KERNEL_LIB = os.path.join(_HERE, "libhprms.so")
BENCH_LIB = os.path.join(_HERE, "libhprms_bench.so")  # bench and tests only, never the product path

HPRMS_OK = 0
HPRMS_E_INVALID = -22
HPRMS_E_LAUNCH = -5
HPRMS_E_RANGE = -34
DTYPE_BF16, DTYPE_FP16 = 0, 1
STREAM_COPY, STREAM_RELU = 0, 1
MAX_PARTS = 8
# the `mode` numbering of hprms_select_config / hprms_kernel_configs
MODE_FUSED, MODE_PLAIN, MODE_FP8, MODE_OUT, MODE_REDUCE, MODE_MXFP8, MODE_MXFP4, MODE_FP8_GROUP = 0, 1, 2, 3, 4, 5, 6, 7
MX_FP8_E4M3, MX_FP4_E2M1 = 0, 1

# every symbol the header declares
SYMBOLS = (
    "hprms_fused_add_rmsnorm",
    "hprms_fused_add_rmsnorm_fp8",
    "hprms_fused_add_rmsnorm_fp8_static",
    "hprms_fused_add_rmsnorm_fp8_group",
    "hprms_fused_add_rmsnorm_fp8_ub",
    "hprms_fused_add_rmsnorm_out",
    "hprms_reduce_add_rmsnorm",
    "hprms_fused_add_rmsnorm_mx",
    "hprms_streamer",
    "hprms_rmsnorm",
    "hprms_fused_add_rmsnorm_config",
    "hprms_select_config",
    "hprms_select_config_cu",
    "hprms_device_cu_count",
    "hprms_set_batch_invariant",
    "hprms_batch_invariant",
    "hprms_kernel_configs",
    "hprms_last_error",
    "hprms_abi_version",
)


class Config(ctypes.Structure):
    _fields_ = [("tier", ctypes.c_int32), ("lanes_per_row", ctypes.c_int32),
                ("vec_per_lane", ctypes.c_int32), ("lds_vec_per_lane", ctypes.c_int32),
                ("block_threads", ctypes.c_int32), ("grid_blocks", ctypes.c_int32),
                ("flags", ctypes.c_int32)]

    def as_tuple(self):
        return tuple(getattr(self, f) for f, _ in self._fields_)


class HprmsError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"{msg} (status {code})")
        self.code = code


def _bind(L, bench):
    vp, i64, ci, cd = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_double
    L.hprms_fused_add_rmsnorm.argtypes = [vp, vp, vp, i64, i64, i64, i64, ci, cd, vp]
    L.hprms_fused_add_rmsnorm_config.argtypes = [vp, vp, vp, i64, i64, i64, i64, ci, cd,
                                                 ctypes.POINTER(Config), vp]
    L.hprms_rmsnorm.argtypes = [vp, vp, vp, i64, i64, i64, i64, ci, cd, vp]
    L.hprms_fused_add_rmsnorm_fp8.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, ci, cd, vp]
    L.hprms_fused_add_rmsnorm_fp8_static.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, ci, cd, vp]
    L.hprms_fused_add_rmsnorm_fp8_ub.argtypes = [vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, ci, cd, vp]
    L.hprms_fused_add_rmsnorm_fp8_group.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, i64, i64, ci, cd,
                                                    vp]
    L.hprms_fused_add_rmsnorm_out.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, i64, ci, cd, vp]
    L.hprms_reduce_add_rmsnorm.argtypes = [vp, ctypes.POINTER(vp), ci, vp, vp, i64, i64, i64, i64, i64, ci,
                                           cd, vp]
    L.hprms_fused_add_rmsnorm_mx.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, i64, ci, ci, cd, vp]
    L.hprms_streamer.argtypes = [vp, vp, i64, i64, i64, i64, ci, ci, vp]
    L.hprms_select_config.argtypes = [i64, i64, ci, ci, ctypes.POINTER(Config)]
    L.hprms_select_config_cu.argtypes = [i64, i64, ci, ci, ci, ctypes.POINTER(Config)]
    L.hprms_device_cu_count.argtypes = [ci]
    L.hprms_set_batch_invariant.argtypes = [ci]
    L.hprms_batch_invariant.argtypes = []
    L.hprms_kernel_configs.argtypes = [ci, ci, ctypes.POINTER(Config), ci]
    L.hprms_last_error.restype = ctypes.c_char_p
    L.hprms_last_error.argtypes = []
    L.hprms_abi_version.restype = ci
    names = ["hprms_fused_add_rmsnorm", "hprms_fused_add_rmsnorm_config", "hprms_rmsnorm",
             "hprms_fused_add_rmsnorm_fp8", "hprms_fused_add_rmsnorm_fp8_static", "hprms_fused_add_rmsnorm_fp8_group",
             "hprms_fused_add_rmsnorm_fp8_ub",
             "hprms_fused_add_rmsnorm_out",
             "hprms_reduce_add_rmsnorm",
             "hprms_fused_add_rmsnorm_mx", "hprms_streamer", "hprms_select_config", "hprms_select_config_cu",
             "hprms_device_cu_count", "hprms_kernel_configs", "hprms_set_batch_invariant", "hprms_batch_invariant"]
    if bench:
        L.hprms_bench_fused_timeline.argtypes = [vp, vp, vp, i64, i64, ci, cd, ctypes.POINTER(Config), vp, vp]
        L.hprms_ceil_empty.argtypes = [i64, ci, vp]
        L.hprms_ceil_read.argtypes = [vp, vp, i64, vp, vp]
        L.hprms_ceil_write.argtypes = [vp, vp, i64, vp]
        L.hprms_ceil_copy.argtypes = [vp, vp, i64, vp]
        L.hprms_ceil_skeleton.argtypes = [vp, vp, i64, i64, ci, ci, ci, ci, vp]
        L.hprms_ceil_streams.argtypes = [ci, vp, vp, vp, vp, i64, vp]
        L.hprms_ceil_flat.argtypes = [ci, ci, ci, ci, vp, vp, i64, vp]
        L.hprms_bench_form_config.argtypes = [ci, vp, vp, i64, i64, vp, vp, vp, i64, i64, ci, cd,
                                              ctypes.POINTER(Config), vp]
        names += ["hprms_bench_fused_timeline", "hprms_bench_form_config", "hprms_ceil_empty", "hprms_ceil_read", "hprms_ceil_write",
                  "hprms_ceil_copy", "hprms_ceil_skeleton", "hprms_ceil_streams", "hprms_ceil_flat"]
    for name in names:
        getattr(L, name).restype = ci


class Library:
    """One build of the C ABI: the product ``libhprms.so`` or the bench
    library ``libhprms_bench.so`` (the same entry points, the tuning-only
    kernel shapes, and the ceiling and timeline entry points)."""

    def __init__(self, path, bench=False):
        self.path = path
        self.bench = bench
        self._L = None

    def lib(self):
        """Load the library.  When torch is importable it is imported first,
        so that the library binds to the HIP runtime torch already loaded."""
        if self._L is None:
            try:
                import torch  # noqa: F401
            except ImportError:
                pass
            if not os.path.exists(self.path):
                raise ImportError(f"{self.path} not built: run `python hp_rms_norm_amd/build.py`")
            L = ctypes.CDLL(self.path)
            _bind(L, self.bench)
            self._L = L
        return self._L

    def last_error(self):
        return self.lib().hprms_last_error().decode()

    def _check(self, rc):
        if rc != HPRMS_OK:
            raise HprmsError(rc, self.last_error())
        return rc

    def fused_add_rmsnorm(self, input_ptr, weight_ptr, residual_ptr, rows, hidden, input_stride, residual_stride,
                          dtype, eps, stream=0, config=None):
        L = self.lib()
        if config is None:
            return self._check(L.hprms_fused_add_rmsnorm(input_ptr, weight_ptr, residual_ptr, rows, hidden,
                                                         input_stride, residual_stride, dtype, eps, stream))
        return self._check(L.hprms_fused_add_rmsnorm_config(input_ptr, weight_ptr, residual_ptr, rows, hidden,
                                                            input_stride, residual_stride, dtype, eps,
                                                            ctypes.byref(config), stream))

    def fused_add_rmsnorm_fp8(self, out_ptr, scale_ptr, input_ptr, weight_ptr, residual_ptr, rows, hidden,
                              out_stride, input_stride, residual_stride, dtype, eps, stream=0):
        return self._check(self.lib().hprms_fused_add_rmsnorm_fp8(out_ptr, scale_ptr, input_ptr, weight_ptr,
                                                                  residual_ptr, rows, hidden, out_stride,
                                                                  input_stride, residual_stride, dtype, eps, stream))

    def fused_add_rmsnorm_fp8_static(self, out_ptr, scale_ptr, input_ptr, weight_ptr, residual_ptr, rows, hidden,
                                     out_stride, input_stride, residual_stride, dtype, eps, stream=0):
        return self._check(self.lib().hprms_fused_add_rmsnorm_fp8_static(
            out_ptr, scale_ptr, input_ptr, weight_ptr, residual_ptr, rows, hidden, out_stride, input_stride,
            residual_stride, dtype, eps, stream))

    def fused_add_rmsnorm_fp8_ub(self, out_ptr, scale_ptr, scale_ub_ptr, input_ptr, weight_ptr, residual_ptr, rows,
                                 hidden, out_stride, input_stride, residual_stride, dtype, eps, stream=0):
        return self._check(self.lib().hprms_fused_add_rmsnorm_fp8_ub(
            out_ptr, scale_ptr, scale_ub_ptr, input_ptr, weight_ptr, residual_ptr, rows, hidden, out_stride,
            input_stride, residual_stride, dtype, eps, stream))

    def fused_add_rmsnorm_fp8_group(self, out_ptr, scales_ptr, input_ptr, weight_ptr, residual_ptr, rows, hidden,
                                    out_stride, scale_stride, scale_group_stride, input_stride, residual_stride,
                                    dtype, eps, stream=0):
        return self._check(self.lib().hprms_fused_add_rmsnorm_fp8_group(
            out_ptr, scales_ptr, input_ptr, weight_ptr, residual_ptr, rows, hidden, out_stride, scale_stride,
            scale_group_stride, input_stride, residual_stride, dtype, eps, stream))

    def fused_add_rmsnorm_out(self, out_ptr, residual_out_ptr, input_ptr, residual_ptr, weight_ptr, rows, hidden,
                              out_stride, residual_out_stride, input_stride, residual_stride, dtype, eps, stream=0):
        return self._check(self.lib().hprms_fused_add_rmsnorm_out(out_ptr, residual_out_ptr, input_ptr,
                                                                  residual_ptr, weight_ptr, rows, hidden, out_stride,
                                                                  residual_out_stride, input_stride, residual_stride,
                                                                  dtype, eps, stream))

    def reduce_add_rmsnorm(self, out_ptr, part_ptrs, weight_ptr, residual_ptr, rows, hidden, out_stride,
                           part_stride, residual_stride, dtype, eps, stream=0):
        """``part_ptrs``: a sequence of device pointers (1 ... MAX_PARTS); a
        ``None`` sequence passes a null array."""
        arr = None if part_ptrs is None else (ctypes.c_void_p * max(1, len(part_ptrs)))(*part_ptrs)
        n = 0 if part_ptrs is None else len(part_ptrs)
        return self._check(self.lib().hprms_reduce_add_rmsnorm(out_ptr, arr, n, weight_ptr, residual_ptr, rows,
                                                               hidden, out_stride, part_stride, residual_stride,
                                                               dtype, eps, stream))

    def fused_add_rmsnorm_mx(self, out_ptr, scales_ptr, input_ptr, weight_ptr, residual_ptr, rows, hidden,
                             out_stride, scale_stride, input_stride, residual_stride, fmt, dtype, eps, stream=0):
        return self._check(self.lib().hprms_fused_add_rmsnorm_mx(out_ptr, scales_ptr, input_ptr, weight_ptr,
                                                                 residual_ptr, rows, hidden, out_stride,
                                                                 scale_stride, input_stride, residual_stride, fmt,
                                                                 dtype, eps, stream))

    def rmsnorm(self, out_ptr, in_ptr, weight_ptr, rows, hidden, out_stride, in_stride, dtype, eps, stream=0):
        return self._check(self.lib().hprms_rmsnorm(out_ptr, in_ptr, weight_ptr, rows, hidden, out_stride,
                                                    in_stride, dtype, eps, stream))

    def streamer(self, out_ptr, in_ptr, rows, hidden, out_stride, in_stride, dtype, op, stream=0):
        return self._check(self.lib().hprms_streamer(out_ptr, in_ptr, rows, hidden, out_stride, in_stride, dtype,
                                                     op, stream))

    def select_config(self, rows, hidden, dtype, mode=0, cus=None):
        """The table's configuration for a MODE_* entry point, on a device of
        `cus` compute units (None: 256, a whole MI355X)."""
        c = Config()
        L = self.lib()
        if cus is None:
            self._check(L.hprms_select_config(rows, hidden, dtype, mode, ctypes.byref(c)))
        else:
            self._check(L.hprms_select_config_cu(rows, hidden, dtype, mode, cus, ctypes.byref(c)))
        return c

    def set_batch_invariant(self, enable):
        """hprms_set_batch_invariant: returns the previous setting."""
        rc = self.lib().hprms_set_batch_invariant(1 if enable else 0)
        if rc < 0:
            raise HprmsError(rc, self.last_error())
        return bool(rc)

    def batch_invariant(self):
        return bool(self.lib().hprms_batch_invariant())

    def device_cu_count(self, device=-1):
        """Compute units of a HIP device (-1: the current one) as the entry
        points use them."""
        n = self.lib().hprms_device_cu_count(device)
        if n < 0:
            raise HprmsError(n, self.last_error())
        return n

    def bench_fused_timeline(self, input_ptr, weight_ptr, residual_ptr, rows, hidden, dtype, eps, config,
                             timeline_ptr, stream=0):
        """Bench library only: the in-place op on contiguous rows with a forced
        configuration carrying flags bit 9 and its timeline buffer."""
        return self._check(self.lib().hprms_bench_fused_timeline(input_ptr, weight_ptr, residual_ptr, rows, hidden,
                                                                 dtype, eps, ctypes.byref(config), timeline_ptr,
                                                                 stream))

    def bench_form_config(self, mode, out_ptr, aux_ptr, aux_stride, aux_group_stride, input_ptr, weight_ptr,
                          residual_ptr, rows, hidden, dtype, eps, config, stream=0):
        """Bench library only: a form of the op (mode 1, 2, 3, 5, 6 or 7) on
        contiguous rows with a forced configuration; `aux` is the residual
        output (mode 3) or the scales."""
        return self._check(self.lib().hprms_bench_form_config(mode, out_ptr, aux_ptr, aux_stride, aux_group_stride,
                                                              input_ptr, weight_ptr, residual_ptr, rows, hidden,
                                                              dtype, eps, ctypes.byref(config), stream))

    def kernel_configs(self, dtype, mode=0):
        """Every vector-tier configuration built for (dtype, mode)."""
        L = self.lib()
        n = L.hprms_kernel_configs(dtype, mode, None, 0)
        if n < 0:
            raise HprmsError(n, self.last_error())
        arr = (Config * n)()
        self._check(0 if L.hprms_kernel_configs(dtype, mode, arr, n) == n else HPRMS_E_INVALID)
        return list(arr)


PRODUCT = Library(KERNEL_LIB)
BENCH = Library(BENCH_LIB, bench=True)


def lib():
    return PRODUCT.lib()


def last_error():
    return PRODUCT.last_error()


fused_add_rmsnorm = PRODUCT.fused_add_rmsnorm
fused_add_rmsnorm_fp8 = PRODUCT.fused_add_rmsnorm_fp8
fused_add_rmsnorm_fp8_static = PRODUCT.fused_add_rmsnorm_fp8_static
fused_add_rmsnorm_fp8_group = PRODUCT.fused_add_rmsnorm_fp8_group
fused_add_rmsnorm_fp8_ub = PRODUCT.fused_add_rmsnorm_fp8_ub
fused_add_rmsnorm_out = PRODUCT.fused_add_rmsnorm_out
reduce_add_rmsnorm = PRODUCT.reduce_add_rmsnorm
fused_add_rmsnorm_mx = PRODUCT.fused_add_rmsnorm_mx
rmsnorm = PRODUCT.rmsnorm
streamer = PRODUCT.streamer
select_config = PRODUCT.select_config
device_cu_count = PRODUCT.device_cu_count
set_batch_invariant = PRODUCT.set_batch_invariant
batch_invariant = PRODUCT.batch_invariant
kernel_configs = PRODUCT.kernel_configs
