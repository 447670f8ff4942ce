"""ctypes access to the kernel C ABI (include/mgb_kernels.h) for kernel-level
parity tests: device buffers plus the histogram, sketch and bin entry points."""
import ctypes
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
LIB_PATH = ROOT / "xgboost-metal_amd" / "python" / "xgboost" / "lib" / "libxgboost.so"


class MgbMatrix(ctypes.Structure):
    _fields_ = [("rows", ctypes.c_uint32), ("cols", ctypes.c_uint32), ("row_stride", ctypes.c_uint32),
                ("bin_bytes", ctypes.c_uint32), ("max_bin", ctypes.c_uint32), ("cut_stride", ctypes.c_uint32),
                ("missing_code", ctypes.c_uint32), ("group_features", ctypes.c_uint32),
                ("group_stride", ctypes.c_uint64)]


class MgbTreeShape(ctypes.Structure):
    _fields_ = [("rows", ctypes.c_uint32), ("cols", ctypes.c_uint32), ("max_bin", ctypes.c_uint32),
                ("max_depth", ctypes.c_uint32), ("rows_per_tile", ctypes.c_uint32),
                ("features_per_group", ctypes.c_uint32), ("unit_hessian", ctypes.c_uint32), ("dense", ctypes.c_uint32),
                ("column_levels", ctypes.c_uint32), ("sparse", ctypes.c_uint32), ("root_rows_per_tile", ctypes.c_uint32),
                ("compact_sampled", ctypes.c_uint32), ("stable_partition", ctypes.c_uint32)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = ctypes.CDLL(str(LIB_PATH))
        _lib.mgb_last_error.restype = ctypes.c_char_p
        _lib.mgb_tree_workspace_bytes.restype = ctypes.c_size_t
    return _lib


def check(rc):
    if rc != 0:
        raise RuntimeError(lib().mgb_last_error().decode())


class Device:
    """A device allocation holding a copy of a numpy array (or zeros)."""

    def __init__(self, nbytes):
        self.ptr = ctypes.c_void_p()
        self.nbytes = max(int(nbytes), 16)
        check(lib().mgb_malloc(ctypes.byref(self.ptr), ctypes.c_size_t(self.nbytes)))
        check(lib().mgb_memset(self.ptr, 0, ctypes.c_size_t(self.nbytes)))

    @classmethod
    def of(cls, array):
        array = np.ascontiguousarray(array)
        d = cls(array.nbytes)
        if array.nbytes:
            check(lib().mgb_memcpy_h2d(d.ptr, array.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(array.nbytes)))
        return d

    def read(self, dtype, count):
        out = np.zeros(count, dtype)
        if out.nbytes:
            check(lib().mgb_memcpy_d2h(out.ctypes.data_as(ctypes.c_void_p), self.ptr, ctypes.c_size_t(out.nbytes)))
        return out

    def __del__(self):
        if getattr(self, "ptr", None) is not None and self.ptr.value:
            lib().mgb_free(self.ptr)
            self.ptr = None


def sketch_cuts(X, max_bin, weights=None):
    X = np.ascontiguousarray(X, np.float32)
    rows, cols = X.shape
    dX = Device.of(X)
    dw = Device.of(np.ascontiguousarray(weights, np.float32)) if weights is not None else None
    dc = Device(cols * max_bin * 4)
    dn = Device(cols * 4)
    check(lib().mgb_sketch_cuts(dX.ptr, ctypes.c_uint32(rows), ctypes.c_uint32(cols), dw.ptr if dw else None,
                                ctypes.c_uint32(max_bin), dc.ptr, dn.ptr))
    return dc.read(np.float32, cols * max_bin).reshape(cols, max_bin), dn.read(np.uint32, cols)


def layout(cols, hist_bins, bin_bytes, G):
    groups = (cols + G - 1) // G
    return groups * G * bin_bytes


def quantize_bins(X, cuts, counts, hist_bins, bin_bytes, G, dense=False, group_major=False):
    """Device bin matrix; `bins` is returned row-major ([rows, groups*G]) for
    either layout."""
    X = np.ascontiguousarray(X, np.float32)
    rows, cols = X.shape
    code = 0xFFFFFFFF if dense else (0xFF if bin_bytes == 1 else 0xFFFF)
    groups = (cols + G - 1) // G
    gbytes = G * bin_bytes
    row_stride, group_stride = (gbytes, rows * gbytes) if group_major else (groups * gbytes, gbytes)
    m = MgbMatrix(rows, cols, row_stride, bin_bytes, hist_bins, cuts.shape[1], code, G, group_stride)
    dX = Device.of(X)
    dcuts = Device.of(np.ascontiguousarray(cuts, np.float32))
    dcounts = Device.of(np.ascontiguousarray(counts, np.uint32))
    dbins = Device(rows * groups * gbytes)
    flag = Device(4)
    check(lib().mgb_quantize_bins(dX.ptr, dcuts.ptr, dcounts.ptr, ctypes.byref(m), dbins.ptr, flag.ptr))
    dtype = np.uint8 if bin_bytes == 1 else np.uint16
    flat = dbins.read(dtype, rows * groups * G)
    if group_major:
        bins = flat.reshape(groups, rows, G).transpose(1, 0, 2).reshape(rows, groups * G)
    else:
        bins = flat.reshape(rows, groups * G)
    return m, dbins, bins, bool(flag.read(np.uint32, 1)[0])


def histogram(m, dbins, rows_list, grad, hess, scales, G, unit=False, rows_per_tile=2048, max_depth=1):
    """Device histogram of a row list: int64 [cols][max_bin+1][2]."""
    gh = np.ascontiguousarray(np.stack([grad, hess], axis=1).astype(np.float32))
    dgh = Device.of(gh)
    dsc = Device.of(np.asarray(scales, np.float32))
    shape = MgbTreeShape(m.rows, m.cols, m.max_bin, max_depth, rows_per_tile, G, 1 if unit else 0, 1)
    ws_bytes = lib().mgb_tree_workspace_bytes(ctypes.byref(shape))
    ws = Device(ws_bytes)
    out = Device(m.cols * (m.max_bin + 1) * 16)
    drows = Device.of(np.ascontiguousarray(rows_list, np.uint32)) if rows_list is not None else None
    count = m.rows if rows_list is None else len(rows_list)
    check(lib().mgb_histogram(ctypes.byref(shape), ctypes.byref(m), dbins.ptr, drows.ptr if drows else None,
                              ctypes.c_uint32(count), dgh.ptr, dsc.ptr, out.ptr, ws.ptr, ctypes.c_size_t(ws_bytes)))
    return out.read(np.int64, m.cols * (m.max_bin + 1) * 2).reshape(m.cols, m.max_bin + 1, 2)


def metric_sum(pred, labels, kind, weights=None, parameter=0.0):
    """mgb_metric_sum on device copies of the inputs."""
    pred = np.ascontiguousarray(pred, np.float32)
    dp, dl = Device.of(pred), Device.of(np.ascontiguousarray(labels, np.float32))
    dw = None if weights is None else Device.of(np.ascontiguousarray(weights, np.float32))
    lib().mgb_metric_workspace_bytes.restype = ctypes.c_size_t
    nbytes = lib().mgb_metric_workspace_bytes(ctypes.c_uint32(pred.size))
    ws = Device(nbytes)
    out = np.zeros(2, np.float32)
    check(lib().mgb_metric_sum(dp.ptr, dl.ptr, dw.ptr if dw else None, ctypes.c_uint32(pred.size),
                               ctypes.c_uint32(kind), ctypes.c_float(parameter), out.ctypes.data_as(ctypes.c_void_p),
                               ws.ptr, ctypes.c_size_t(ws.nbytes)))
    return out


def metric_auc(pred, labels, pr=False, weights=None):
    pred = np.ascontiguousarray(pred, np.float32)
    dp, dl = Device.of(pred), Device.of(np.ascontiguousarray(labels, np.float32))
    dw = None if weights is None else Device.of(np.ascontiguousarray(weights, np.float32))
    lib().mgb_metric_workspace_bytes.restype = ctypes.c_size_t
    ws = Device(lib().mgb_metric_workspace_bytes(ctypes.c_uint32(pred.size)))
    out = np.zeros(3, np.float64)
    check(lib().mgb_metric_auc(dp.ptr, dl.ptr, dw.ptr if dw else None, ctypes.c_uint32(pred.size), ctypes.c_int(int(pr)),
                               out.ctypes.data_as(ctypes.c_void_p), ws.ptr, ctypes.c_size_t(ws.nbytes)))
    return out
