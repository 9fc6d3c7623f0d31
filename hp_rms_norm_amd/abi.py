"""ctypes binding of the C ABI of ``libhprms.so`` (include/hp_rms_norm_amd.h).

This is the binding a caller without the torch extension would use; the
tests use it to drive the kernels through the C ABI directly.  Device
pointers and streams are plain integers (e.g. ``tensor.data_ptr()`` and
``torch.cuda.current_stream().cuda_stream``).
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
KERNEL_LIB = os.path.join(_HERE, "libhprms.so")

HPRMS_OK = 0
HPRMS_E_INVALID = -22
HPRMS_E_LAUNCH = -5
HPRMS_E_RANGE = -34
DTYPE_BF16, DTYPE_FP16 = 0, 1
STREAM_COPY, STREAM_RELU = 0, 1
MAX_PARTS = 8
# the `mode` numbering of hprms_select_config / hprms_kernel_configs
MODE_FUSED, MODE_PLAIN, MODE_FP8, MODE_OUT, MODE_REDUCE, MODE_MXFP8, MODE_MXFP4 = 0, 1, 2, 3, 4, 5, 6
MX_FP8_E4M3, MX_FP4_E2M1 = 0, 1

# every symbol the header declares
SYMBOLS = (
    "hprms_fused_add_rmsnorm",
    "hprms_fused_add_rmsnorm_fp8",
    "hprms_fused_add_rmsnorm_out",
    "hprms_reduce_add_rmsnorm",
    "hprms_fused_add_rmsnorm_mx",
    "hprms_streamer",
    "hprms_rmsnorm",
    "hprms_fused_add_rmsnorm_config",
    "hprms_select_config",
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


_lib = None


def lib():
    """Load libhprms.so.  When torch is importable it is imported first, so
    that the library binds to the HIP runtime torch already loaded."""
    global _lib
    if _lib is None:
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        if not os.path.exists(KERNEL_LIB):
            raise ImportError(f"{KERNEL_LIB} not built: run `python hp_rms_norm_amd/build.py`")
        L = ctypes.CDLL(KERNEL_LIB)
        vp, i64, ci, cd = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_double
        L.hprms_fused_add_rmsnorm.argtypes = [vp, vp, vp, i64, i64, i64, i64, ci, cd, vp]
        L.hprms_fused_add_rmsnorm_config.argtypes = [vp, vp, vp, i64, i64, i64, i64, ci, cd,
                                                     ctypes.POINTER(Config), vp]
        L.hprms_rmsnorm.argtypes = [vp, vp, vp, i64, i64, i64, i64, ci, cd, vp]
        L.hprms_fused_add_rmsnorm_fp8.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, ci, cd, vp]
        L.hprms_fused_add_rmsnorm_out.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, i64, ci, cd, vp]
        L.hprms_reduce_add_rmsnorm.argtypes = [vp, ctypes.POINTER(vp), ci, vp, vp, i64, i64, i64, i64, i64, ci,
                                               cd, vp]
        L.hprms_fused_add_rmsnorm_mx.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, i64, ci, ci, cd, vp]
        L.hprms_streamer.argtypes = [vp, vp, i64, i64, i64, i64, ci, ci, vp]
        L.hprms_select_config.argtypes = [i64, i64, ci, ci, ctypes.POINTER(Config)]
        L.hprms_kernel_configs.argtypes = [ci, ci, ctypes.POINTER(Config), ci]
        L.hprms_last_error.restype = ctypes.c_char_p
        L.hprms_last_error.argtypes = []
        L.hprms_abi_version.restype = ci
        for name in ("hprms_fused_add_rmsnorm", "hprms_fused_add_rmsnorm_config", "hprms_rmsnorm",
                     "hprms_fused_add_rmsnorm_fp8", "hprms_fused_add_rmsnorm_out", "hprms_reduce_add_rmsnorm",
                     "hprms_fused_add_rmsnorm_mx",
                     "hprms_streamer", "hprms_select_config", "hprms_kernel_configs"):
            getattr(L, name).restype = ci
        _lib = L
    return _lib


def last_error():
    return lib().hprms_last_error().decode()


def _check(rc):
    if rc != HPRMS_OK:
        raise HprmsError(rc, last_error())
    return rc


def fused_add_rmsnorm(input_ptr, weight_ptr, residual_ptr, rows, hidden, input_stride, residual_stride,
                      dtype, eps, stream=0, config=None):
    if config is None:
        return _check(lib().hprms_fused_add_rmsnorm(input_ptr, weight_ptr, residual_ptr, rows, hidden,
                                                    input_stride, residual_stride, dtype, eps, stream))
    return _check(lib().hprms_fused_add_rmsnorm_config(input_ptr, weight_ptr, residual_ptr, rows, hidden,
                                                       input_stride, residual_stride, dtype, eps,
                                                       ctypes.byref(config), stream))


def fused_add_rmsnorm_fp8(out_ptr, scale_ptr, input_ptr, weight_ptr, residual_ptr, rows, hidden, out_stride,
                          input_stride, residual_stride, dtype, eps, stream=0):
    return _check(lib().hprms_fused_add_rmsnorm_fp8(out_ptr, scale_ptr, input_ptr, weight_ptr, residual_ptr, rows,
                                                    hidden, out_stride, input_stride, residual_stride, dtype, eps,
                                                    stream))


def fused_add_rmsnorm_out(out_ptr, residual_out_ptr, input_ptr, residual_ptr, weight_ptr, rows, hidden,
                          out_stride, residual_out_stride, input_stride, residual_stride, dtype, eps, stream=0):
    return _check(lib().hprms_fused_add_rmsnorm_out(out_ptr, residual_out_ptr, input_ptr, residual_ptr, weight_ptr,
                                                    rows, hidden, out_stride, residual_out_stride, input_stride,
                                                    residual_stride, dtype, eps, stream))


def reduce_add_rmsnorm(out_ptr, part_ptrs, weight_ptr, residual_ptr, rows, hidden, out_stride, part_stride,
                       residual_stride, dtype, eps, stream=0):
    """``part_ptrs``: a sequence of device pointers (1 ... MAX_PARTS); a
    ``None`` sequence passes a null array."""
    arr = None if part_ptrs is None else (ctypes.c_void_p * max(1, len(part_ptrs)))(*part_ptrs)
    n = 0 if part_ptrs is None else len(part_ptrs)
    return _check(lib().hprms_reduce_add_rmsnorm(out_ptr, arr, n, weight_ptr, residual_ptr, rows, hidden, out_stride,
                                                 part_stride, residual_stride, dtype, eps, stream))


def fused_add_rmsnorm_mx(out_ptr, scales_ptr, input_ptr, weight_ptr, residual_ptr, rows, hidden, out_stride,
                         scale_stride, input_stride, residual_stride, fmt, dtype, eps, stream=0):
    return _check(lib().hprms_fused_add_rmsnorm_mx(out_ptr, scales_ptr, input_ptr, weight_ptr, residual_ptr, rows,
                                                   hidden, out_stride, scale_stride, input_stride, residual_stride,
                                                   fmt, dtype, eps, stream))


def rmsnorm(out_ptr, in_ptr, weight_ptr, rows, hidden, out_stride, in_stride, dtype, eps, stream=0):
    return _check(lib().hprms_rmsnorm(out_ptr, in_ptr, weight_ptr, rows, hidden, out_stride, in_stride,
                                      dtype, eps, stream))


def streamer(out_ptr, in_ptr, rows, hidden, out_stride, in_stride, dtype, op, stream=0):
    return _check(lib().hprms_streamer(out_ptr, in_ptr, rows, hidden, out_stride, in_stride, dtype, op,
                                       stream))


def select_config(rows, hidden, dtype, mode=0):
    """The table's configuration for a MODE_* entry point."""
    c = Config()
    _check(lib().hprms_select_config(rows, hidden, dtype, mode, ctypes.byref(c)))
    return c


def kernel_configs(dtype, mode=0):
    """Every vector-tier configuration built for (dtype, mode)."""
    n = lib().hprms_kernel_configs(dtype, mode, None, 0)
    if n < 0:
        raise HprmsError(n, last_error())
    arr = (Config * n)()
    _check(0 if lib().hprms_kernel_configs(dtype, mode, arr, n) == n else HPRMS_E_INVALID)
    return list(arr)
