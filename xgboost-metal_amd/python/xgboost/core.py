"""Core data structures of the HIP hist engine: DMatrix, QuantileDMatrix, Booster.

Counterpart of the reference's python-package/xgboost/core.py (DMatrix
:676, QuantileDMatrix :1476, Booster :1796) over the C API declared in
include/xgboost_c_api.h.  Data is passed as numpy __array_interface__ JSON,
as upstream XGBoost does.
"""
from __future__ import annotations

import ctypes
import json
import os
import weakref
from abc import ABC, abstractmethod
from typing import Any, Callable, Dict, Iterable, List, Optional, Sequence, Tuple, Union

import numpy as np

from .libpath import find_lib_path

c_bst_ulong = ctypes.c_uint64


class XGBoostError(ValueError):
    """Error raised by the native library."""


def _load_lib():
    path = find_lib_path()
    lib = ctypes.cdll.LoadLibrary(path)
    lib.XGBGetLastError.restype = ctypes.c_char_p
    major, minor, patch = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    lib.XGBoostVersion(ctypes.byref(major), ctypes.byref(minor), ctypes.byref(patch))
    if (major.value, minor.value) != (3, 5):
        raise XGBoostError(f"libxgboost version {major.value}.{minor.value} does not match the package (3.5)")
    lib.path = path
    return lib


_LIB = _load_lib()


def _check_call(ret: int) -> None:
    if ret != 0:
        raise XGBoostError(_LIB.XGBGetLastError().decode())


def c_str(s: str) -> ctypes.c_char_p:
    return ctypes.c_char_p(s.encode("utf-8"))


def build_info() -> dict:
    out = ctypes.c_char_p()
    _check_call(_LIB.XGBuildInfo(ctypes.byref(out)))
    info = json.loads(out.value.decode())
    info["libxgboost"] = _LIB.path
    return info


def _array_interface(a: np.ndarray) -> bytes:
    inter = dict(a.__array_interface__)
    if "mask" in inter:
        del inter["mask"]
    inter["data"] = [int(inter["data"][0]), bool(inter["data"][1])]
    if inter.get("strides") is not None:
        inter["strides"] = list(inter["strides"])
    inter["shape"] = list(inter["shape"])
    inter.pop("descr", None)
    return json.dumps(inter).encode()


def _to_numpy_2d(data: Any) -> np.ndarray:
    if hasattr(data, "to_numpy") and hasattr(data, "columns"):  # pandas DataFrame
        data = data.to_numpy(dtype=np.float32, na_value=np.nan)
    arr = np.asarray(data)
    if arr.ndim == 1:
        arr = arr.reshape(-1, 1)
    if arr.ndim != 2:
        raise ValueError("data must be 2-dimensional")
    if arr.dtype == np.float64 or arr.dtype == np.float16 or arr.dtype.kind in "iub" or arr.dtype == object:
        arr = arr.astype(np.float32)
    elif arr.dtype != np.float32:
        arr = arr.astype(np.float32)
    return arr


def _is_scipy_csr(data: Any) -> bool:
    return type(data).__name__ in ("csr_matrix", "csr_array")


def _feature_names_of(data: Any) -> Optional[List[str]]:
    if hasattr(data, "columns"):
        return [str(c) for c in data.columns]
    return None


def _missing_value(missing: Optional[float]) -> Optional[float]:
    return None if missing is None or np.isnan(missing) else float(missing)


class DataIter(ABC):
    """User-defined batch iterator (the reference's core.py:275 interface).

    ``next(input_data)`` passes one batch by calling
    ``input_data(data=..., label=..., weight=..., ...)`` and returns True, or
    returns False after the last batch; ``reset()`` rewinds.  The engine
    concatenates the batches in host memory, so ``cache_prefix`` (external
    memory) is rejected.  An exception raised in ``next`` or ``reset`` ends the
    iteration and is raised again when the DMatrix construction returns.
    """

    def __init__(self, cache_prefix: Optional[str] = None, release_data: bool = True, *, on_host: bool = True,
                 min_cache_page_bytes: Optional[int] = None) -> None:
        self.cache_prefix = cache_prefix
        self.on_host = on_host
        self.min_cache_page_bytes = min_cache_page_bytes
        self.release_data = release_data
        self._proxy = _ProxyDMatrix()

    @property
    def proxy(self) -> "_ProxyDMatrix":
        """The proxy matrix each batch is staged in for the C library."""
        return self._proxy

    @abstractmethod
    def reset(self) -> None:
        """Rewind the iterator."""
        raise NotImplementedError()

    @abstractmethod
    def next(self, input_data: Callable) -> bool:
        """Pass the next batch to ``input_data``; False when there is none."""
        raise NotImplementedError()


_RESET_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p)
_NEXT_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p)


class _IterationBridge:
    """One C call that pulls a DataIter's batches through reset/next
    function pointers.

    A Python exception cannot unwind through the library's C frames: the
    first one raised by the iterator is stored, every later callback answers
    "no more batches", and ``call`` raises it once the C function has
    returned.  The current batch's arrays stay referenced until the library
    has copied them (the next callback, or the end of the call when the
    iterator keeps its data)."""

    def __init__(self, it: DataIter) -> None:
        self._it = it
        self._failure: Optional[BaseException] = None
        self._staged: Any = None
        self._reset_fn = _RESET_FN(self._on_reset)
        self._next_fn = _NEXT_FN(self._on_next)

    def _guarded(self, action: Callable[[], Any], on_failure: Any) -> Any:
        if self._failure is not None:
            return on_failure
        try:
            return action()
        except Exception as failure:  # pylint: disable=broad-except
            self._failure = failure
            return on_failure

    def _on_reset(self, _context: Any) -> None:
        if self._it.release_data:
            self._staged = None
        self._guarded(self._it.reset, None)

    def _on_next(self, _context: Any) -> int:
        if self._it.release_data:
            self._staged = None
        return self._guarded(lambda: 1 if self._it.next(self._stage) else 0, 0)

    def _stage(self, *, data: Any, feature_names: Optional[Sequence[str]] = None,
               feature_types: Optional[Sequence[str]] = None, **info: Any) -> None:
        proxy = self._it.proxy
        self._staged = proxy._set_data(data)
        proxy.set_info(feature_names=_feature_names_of(data) if feature_names is None else feature_names,
                       feature_types=feature_types, **info)

    def call(self, invoke: Callable[[Any, Any], int]) -> int:
        """invoke(reset, next) calls the C function with the two function
        pointers; the iterator's first exception, if any, is raised after it
        returns."""
        try:
            ret = invoke(self._reset_fn, self._next_fn)
        finally:
            self._staged = None
        if self._failure is not None:
            failure, self._failure = self._failure, None
            raise failure
        return ret


class _SingleBatchIter(DataIter):
    """One in-memory batch as an iterator (QuantileDMatrix with ``ref``)."""

    def __init__(self, **kwargs: Any) -> None:
        self._kwargs = kwargs
        self._done = False
        super().__init__(release_data=False)

    def next(self, input_data: Callable) -> bool:
        if self._done:
            return False
        self._done = True
        input_data(**self._kwargs)
        return True

    def reset(self) -> None:
        self._done = False


class DMatrix:
    """Data matrix for training and prediction (reference core.py:676)."""

    def __init__(self, data: Any, label: Any = None, *, weight: Any = None, base_margin: Any = None,
                 missing: Optional[float] = None, silent: bool = False, feature_names: Optional[Sequence[str]] = None,
                 feature_types: Optional[Sequence[str]] = None, nthread: Optional[int] = None,
                 enable_categorical: bool = False, **kwargs: Any) -> None:
        if isinstance(data, ctypes.c_void_p):
            # A handle the C API returned (slices).
            self.handle = data
            return
        self.handle = ctypes.c_void_p()
        if isinstance(data, DataIter):
            self._init_from_iter(data, missing)
            self.set_info(label=label, weight=weight, base_margin=base_margin, feature_names=feature_names,
                          feature_types=feature_types)
            return
        self._init(data, missing, kwargs.pop("_config", None))
        if feature_names is None:
            feature_names = _feature_names_of(data)
        self.set_info(label=label, weight=weight, base_margin=base_margin, feature_names=feature_names,
                      feature_types=feature_types)

    def _init(self, data: Any, missing: Optional[float], extra: Optional[dict]) -> None:
        config = {"missing": None if missing is None or np.isnan(missing) else float(missing), "nthread": 0}
        if extra:
            config.update(extra)
        cfg = json.dumps(config).encode()
        if _is_scipy_csr(data):
            csr = data
            indptr = np.ascontiguousarray(csr.indptr, dtype=np.int64)
            indices = np.ascontiguousarray(csr.indices, dtype=np.int32)
            values = np.ascontiguousarray(csr.data, dtype=np.float32)
            self._keep = (indptr, indices, values)
            _check_call(_LIB.XGDMatrixCreateFromCSR(_array_interface(indptr), _array_interface(indices),
                                                    _array_interface(values), c_bst_ulong(csr.shape[1]), cfg,
                                                    ctypes.byref(self.handle)))
            return
        if type(data).__name__ in ("csc_matrix", "csc_array", "coo_matrix", "coo_array"):
            self._init(data.tocsr(), missing, extra)
            return
        arr = _to_numpy_2d(data)
        _check_call(_LIB.XGDMatrixCreateFromDense(_array_interface(arr), cfg, ctypes.byref(self.handle)))

    def _init_from_iter(self, it: "DataIter", missing: Optional[float]) -> None:
        """Concatenate an iterator's batches in memory (reference core.py:862)."""
        if it.cache_prefix:
            raise XGBoostError("External memory (cache_prefix) is not supported by this engine")
        config = json.dumps({"missing": _missing_value(missing), "cache_prefix": "", "nthread": 0}).encode()
        _check_call(_IterationBridge(it).call(lambda reset, nxt: _LIB.XGDMatrixCreateFromCallback(
            None, it.proxy.handle, reset, nxt, config, ctypes.byref(self.handle))))

    def __del__(self) -> None:
        if getattr(self, "handle", None) is not None and self.handle.value:
            _check_call(_LIB.XGDMatrixFree(self.handle))
            self.handle = None

    def slice(self, rindex: Union[List[int], np.ndarray], allow_groups: bool = False) -> "DMatrix":
        """A new DMatrix holding the rows ``rindex`` (reference core.py:1264)."""
        idx = np.ascontiguousarray(np.asarray(rindex, dtype=np.int32).reshape(-1))
        handle = ctypes.c_void_p()
        _check_call(_LIB.XGDMatrixSliceDMatrixEx(self.handle, idx.ctypes.data_as(ctypes.POINTER(ctypes.c_int)),
                                                 c_bst_ulong(idx.size), ctypes.byref(handle),
                                                 ctypes.c_int(1 if allow_groups else 0)))
        return DMatrix(handle)

    def get_data(self) -> Any:
        """The predictors as a scipy CSR matrix of the stored values (reference core.py:1122)."""
        import scipy.sparse

        nnz = self.num_nonmissing()
        indptr = np.empty(self.num_row() + 1, dtype=np.uint64)
        indices = np.empty(nnz, dtype=np.uint32)
        data = np.empty(nnz, dtype=np.float32)
        _check_call(_LIB.XGDMatrixGetDataAsCSR(self.handle, b"{}", indptr.ctypes.data_as(ctypes.POINTER(c_bst_ulong)),
                                               indices.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                                               data.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))
        return scipy.sparse.csr_matrix((data, indices, indptr), shape=(self.num_row(), self.num_col()))

    def save_binary(self, fname: Union[str, os.PathLike], silent: bool = True) -> None:
        _check_call(_LIB.XGDMatrixSaveBinary(self.handle, c_str(os.fspath(fname)), ctypes.c_int(silent)))

    # ---- info ----------------------------------------------------------------
    def set_info(self, *, label: Any = None, weight: Any = None, base_margin: Any = None,
                 feature_names: Optional[Sequence[str]] = None, feature_types: Optional[Sequence[str]] = None,
                 **kwargs: Any) -> None:
        if label is not None:
            self.set_label(label)
        if weight is not None:
            self.set_weight(weight)
        if base_margin is not None:
            self.set_base_margin(base_margin)
        if feature_names is not None:
            self.feature_names = list(feature_names)
        if feature_types is not None:
            self.feature_types = list(feature_types)
        for key, value in kwargs.items():
            if value is not None:
                self.set_float_info(key, value)

    def set_float_info(self, field: str, data: Any) -> None:
        arr = np.ascontiguousarray(np.asarray(data, dtype=np.float32).reshape(-1))
        _check_call(_LIB.XGDMatrixSetInfoFromInterface(self.handle, c_str(field), _array_interface(arr)))

    def get_float_info(self, field: str) -> np.ndarray:
        length = c_bst_ulong()
        ptr = ctypes.POINTER(ctypes.c_float)()
        _check_call(_LIB.XGDMatrixGetFloatInfo(self.handle, c_str(field), ctypes.byref(length), ctypes.byref(ptr)))
        if length.value == 0:
            return np.zeros(0, np.float32)
        return np.ctypeslib.as_array(ptr, shape=(length.value,)).copy()

    def set_label(self, label: Any) -> None:
        if hasattr(label, "to_numpy"):
            label = label.to_numpy()
        self.set_float_info("label", label)

    def set_weight(self, weight: Any) -> None:
        self.set_float_info("weight", weight)

    def set_base_margin(self, margin: Any) -> None:
        self.set_float_info("base_margin", margin)

    def get_label(self) -> np.ndarray:
        return self.get_float_info("label")

    def get_weight(self) -> np.ndarray:
        return self.get_float_info("weight")

    def get_base_margin(self) -> np.ndarray:
        return self.get_float_info("base_margin")

    def num_row(self) -> int:
        out = c_bst_ulong()
        _check_call(_LIB.XGDMatrixNumRow(self.handle, ctypes.byref(out)))
        return out.value

    def num_col(self) -> int:
        out = c_bst_ulong()
        _check_call(_LIB.XGDMatrixNumCol(self.handle, ctypes.byref(out)))
        return out.value

    def num_nonmissing(self) -> int:
        out = c_bst_ulong()
        _check_call(_LIB.XGDMatrixNumNonMissing(self.handle, ctypes.byref(out)))
        return out.value

    def _get_str_info(self, field: str) -> Optional[List[str]]:
        size = c_bst_ulong()
        ptr = ctypes.POINTER(ctypes.c_char_p)()
        _check_call(_LIB.XGDMatrixGetStrFeatureInfo(self.handle, c_str(field), ctypes.byref(size), ctypes.byref(ptr)))
        if size.value == 0:
            return None
        return [ptr[i].decode() for i in range(size.value)]

    def _set_str_info(self, field: str, values: Optional[Sequence[str]]) -> None:
        values = [] if values is None else [str(v) for v in values]
        if values and len(values) != self.num_col():
            raise ValueError(f"{field} must have one entry per feature")
        arr = (ctypes.c_char_p * len(values))(*[v.encode() for v in values])
        _check_call(_LIB.XGDMatrixSetStrFeatureInfo(self.handle, c_str(field), arr, c_bst_ulong(len(values))))

    @property
    def feature_names(self) -> Optional[List[str]]:
        return self._get_str_info("feature_name")

    @feature_names.setter
    def feature_names(self, names: Optional[Sequence[str]]) -> None:
        if names is not None and len(set(names)) != len(names):
            raise ValueError("feature_names must be unique")
        self._set_str_info("feature_name", names)

    @property
    def feature_types(self) -> Optional[List[str]]:
        return self._get_str_info("feature_type")

    @feature_types.setter
    def feature_types(self, types: Optional[Sequence[str]]) -> None:
        self._set_str_info("feature_type", types)

    def to_device(self) -> "DMatrix":
        """Engine extension: copy the values, labels and weights to the GPU now
        (otherwise done when training or prediction first needs them)."""
        _check_call(_LIB.XGDMatrixHipUpload(self.handle))
        return self

    def get_quantile_cut(self) -> Tuple[np.ndarray, np.ndarray]:
        """Histogram cut points: (indptr, values) per feature."""
        indptr = ctypes.c_char_p()
        values = ctypes.c_char_p()
        _check_call(_LIB.XGDMatrixGetQuantileCut(self.handle, b"{}", ctypes.byref(indptr), ctypes.byref(values)))
        return _from_interface(indptr.value), _from_interface(values.value)


class _ProxyDMatrix(DMatrix):
    """Staging matrix an iterator fills one batch at a time (reference core.py:1430).

    The C side copies each batch when it is set.
    """

    def __init__(self) -> None:  # pylint: disable=super-init-not-called
        self.handle = ctypes.c_void_p()
        _check_call(_LIB.XGProxyDMatrixCreate(ctypes.byref(self.handle)))

    def _set_data(self, data: Any) -> Any:
        if type(data).__name__ in ("csc_matrix", "csc_array", "coo_matrix", "coo_array"):
            data = data.tocsr()
        if _is_scipy_csr(data):
            indptr = np.ascontiguousarray(data.indptr, dtype=np.int64)
            indices = np.ascontiguousarray(data.indices, dtype=np.int32)
            values = np.ascontiguousarray(data.data, dtype=np.float32)
            _check_call(_LIB.XGProxyDMatrixSetDataCSR(self.handle, _array_interface(indptr),
                                                      _array_interface(indices), _array_interface(values),
                                                      c_bst_ulong(data.shape[1])))
            return indptr, indices, values
        arr = _to_numpy_2d(data)
        _check_call(_LIB.XGProxyDMatrixSetDataDense(self.handle, _array_interface(arr)))
        return arr


def _from_interface(text: bytes) -> np.ndarray:
    inter = json.loads(text)
    n = inter["shape"][0]
    dtype = np.dtype(inter["typestr"])
    if n == 0:
        return np.zeros(0, dtype)
    buf = (ctypes.c_char * (n * dtype.itemsize)).from_address(inter["data"][0])
    return np.frombuffer(buf, dtype=dtype, count=n).copy()


class QuantileDMatrix(DMatrix):
    """DMatrix quantized at construction with ``max_bin`` (reference core.py:1476).

    Training with a different ``max_bin`` is an error, as in XGBoost.
    """

    def __init__(self, data: Any, label: Any = None, *, weight: Any = None, base_margin: Any = None,
                 missing: Optional[float] = None, silent: bool = False, feature_names: Optional[Sequence[str]] = None,
                 feature_types: Optional[Sequence[str]] = None, nthread: Optional[int] = None, max_bin: int = 256,
                 ref: Optional[DMatrix] = None, enable_categorical: bool = False, **kwargs: Any) -> None:
        self.max_bin = int(max_bin)
        if isinstance(data, ctypes.c_void_p):
            self.handle = data
            return
        if isinstance(data, DataIter) or ref is not None:
            # Iterator path (reference core.py:1620-1660): batches are
            # concatenated; ``ref`` makes this matrix use the cuts of the
            # reference matrix instead of sketching its own.
            it = data
            if not isinstance(it, DataIter):
                it = _SingleBatchIter(data=data, label=label, weight=weight, base_margin=base_margin,
                                      feature_names=feature_names if feature_names is not None
                                      else _feature_names_of(data), feature_types=feature_types)
                label = weight = base_margin = None
                feature_names = feature_types = None
            if it.cache_prefix:
                raise XGBoostError("External memory (cache_prefix) is not supported by this engine")
            self.handle = ctypes.c_void_p()
            config = json.dumps({"missing": _missing_value(missing), "nthread": 0, "max_bin": self.max_bin}).encode()
            ref_handle = ref.handle if ref is not None else None
            _check_call(_IterationBridge(it).call(lambda reset, nxt: _LIB.XGQuantileDMatrixCreateFromCallback(
                None, it.proxy.handle, ref_handle, reset, nxt, config, ctypes.byref(self.handle))))
            self.set_info(label=label, weight=weight, base_margin=base_margin, feature_names=feature_names,
                          feature_types=feature_types)
            return
        super().__init__(data, label, weight=weight, base_margin=base_margin, missing=missing,
                         feature_names=feature_names, feature_types=feature_types,
                         _config={"max_bin": self.max_bin, "quantile": True})


def _params_items(params: Any) -> List[Tuple[str, Any]]:
    if params is None:
        return []
    if isinstance(params, dict):
        return list(params.items())
    return list(params)


def _param_value(value: Any) -> str:
    if isinstance(value, bool):
        return "1" if value else "0"
    if isinstance(value, (list, tuple)):
        return json.dumps(list(value))
    if isinstance(value, float):
        return repr(value)
    return str(value)


class Booster:
    """A gradient-boosted tree model (reference core.py:1796)."""

    def __init__(self, params: Optional[Dict[str, Any]] = None, cache: Optional[Sequence[DMatrix]] = None,
                 model_file: Union[str, os.PathLike, bytearray, "Booster", None] = None) -> None:
        cache = list(cache) if cache is not None else []
        handles = (ctypes.c_void_p * len(cache))(*[d.handle for d in cache])
        self.handle = ctypes.c_void_p()
        _check_call(_LIB.XGBoosterCreate(handles, c_bst_ulong(len(cache)), ctypes.byref(self.handle)))
        self.feature_names = None
        self.feature_types = None
        if cache:
            self.feature_names = cache[0].feature_names
            self.feature_types = cache[0].feature_types
        if isinstance(model_file, Booster):
            # A memory snapshot of the other booster (model, configuration and
            # random-engine state), as upstream's copy does.
            state = model_file.__getstate__()
            raw = state["raw"]
            buf = (ctypes.c_char * len(raw)).from_buffer_copy(raw)
            _check_call(_LIB.XGBoosterUnserializeFromBuffer(self.handle, buf, c_bst_ulong(len(raw))))
            self.feature_names = state.get("feature_names")
            self.feature_types = state.get("feature_types")
        elif model_file is not None:
            self.load_model(model_file)
        self.set_param(params or {})

    def __del__(self) -> None:
        if getattr(self, "handle", None) is not None and self.handle.value:
            _check_call(_LIB.XGBoosterFree(self.handle))
            self.handle = None

    def __getstate__(self) -> dict:
        length = c_bst_ulong()
        ptr = ctypes.POINTER(ctypes.c_char)()
        _check_call(_LIB.XGBoosterSerializeToBuffer(self.handle, ctypes.byref(length), ctypes.byref(ptr)))
        return {"raw": bytes(ctypes.string_at(ptr, length.value)), "feature_names": self.feature_names,
                "feature_types": self.feature_types}

    def __setstate__(self, state: dict) -> None:
        self.handle = ctypes.c_void_p()
        _check_call(_LIB.XGBoosterCreate(None, c_bst_ulong(0), ctypes.byref(self.handle)))
        raw = state["raw"]
        buf = (ctypes.c_char * len(raw)).from_buffer_copy(raw)
        _check_call(_LIB.XGBoosterUnserializeFromBuffer(self.handle, buf, c_bst_ulong(len(raw))))
        self.feature_names = state.get("feature_names")
        self.feature_types = state.get("feature_types")

    def __copy__(self) -> "Booster":
        return self.copy()

    def copy(self) -> "Booster":
        return Booster(model_file=self)

    def reset(self) -> "Booster":
        _check_call(_LIB.XGBoosterReset(self.handle))
        return self

    # ---- parameters ----------------------------------------------------------
    def set_param(self, params: Any, value: Optional[str] = None) -> None:
        if isinstance(params, str) and value is not None:
            params = [(params, value)]
        for key, val in _params_items(params):
            if val is None:
                continue
            if key == "monotone_constraints" and isinstance(val, dict):
                # Constraints by feature name (reference core.py Booster
                # _configure_constraints): one entry per training feature, in order.
                names = self.feature_names
                if names is None or not set(val).issubset(names):
                    raise ValueError("Constrained features are not a subset of training data feature names")
                val = tuple(int(val.get(name, 0)) for name in names)
            if key == "eval_metric" and isinstance(val, (list, tuple)):
                # Each listed metric is one eval_metric setting, in order.
                for metric in val:
                    _check_call(_LIB.XGBoosterSetParam(self.handle, c_str("eval_metric"), c_str(str(metric))))
                continue
            _check_call(_LIB.XGBoosterSetParam(self.handle, c_str(str(key)), c_str(_param_value(val))))

    def attr(self, key: str) -> Optional[str]:
        out = ctypes.c_char_p()
        ok = ctypes.c_int()
        _check_call(_LIB.XGBoosterGetAttr(self.handle, c_str(key), ctypes.byref(out), ctypes.byref(ok)))
        return out.value.decode() if ok.value else None

    def attributes(self) -> Dict[str, Optional[str]]:
        length = c_bst_ulong()
        ptr = ctypes.POINTER(ctypes.c_char_p)()
        _check_call(_LIB.XGBoosterGetAttrNames(self.handle, ctypes.byref(length), ctypes.byref(ptr)))
        names = [ptr[i].decode() for i in range(length.value)]
        return {n: self.attr(n) for n in names}

    def set_attr(self, **kwargs: Optional[str]) -> None:
        for key, value in kwargs.items():
            _check_call(_LIB.XGBoosterSetAttr(self.handle, c_str(key),
                                              None if value is None else c_str(str(value))))

    # ---- training --------------------------------------------------------------
    def update(self, dtrain: DMatrix, iteration: int, fobj: Any = None) -> None:
        if not isinstance(dtrain, DMatrix):
            raise TypeError("invalid training matrix")
        if fobj is None:
            _check_call(_LIB.XGBoosterUpdateOneIter(self.handle, ctypes.c_int(iteration), dtrain.handle))
        else:
            pred = self.predict(dtrain, output_margin=True, training=True)
            grad, hess = fobj(pred, dtrain)
            self.boost(dtrain, iteration, grad, hess)

    def boost(self, dtrain: DMatrix, iteration: int, grad: Any, hess: Any) -> None:
        g = np.ascontiguousarray(np.asarray(grad, dtype=np.float32).reshape(-1))
        h = np.ascontiguousarray(np.asarray(hess, dtype=np.float32).reshape(-1))
        if g.shape != h.shape:
            raise ValueError("grad and hess must have the same shape")
        _check_call(_LIB.XGBoosterTrainOneIter(self.handle, dtrain.handle, ctypes.c_int(iteration),
                                               _array_interface(g), _array_interface(h)))

    def eval_set(self, evals: Sequence[Tuple[DMatrix, str]], iteration: int = 0, feval: Any = None,
                 output_margin: bool = True) -> str:
        handles = (ctypes.c_void_p * len(evals))(*[d.handle for d, _ in evals])
        names = (ctypes.c_char_p * len(evals))(*[n.encode() for _, n in evals])
        out = ctypes.c_char_p()
        _check_call(_LIB.XGBoosterEvalOneIter(self.handle, ctypes.c_int(iteration), handles, names,
                                              c_bst_ulong(len(evals)), ctypes.byref(out)))
        result = out.value.decode()
        if feval is not None:
            for dmat, name in evals:
                feval_ret = feval(self.predict(dmat, output_margin=output_margin), dmat)
                if isinstance(feval_ret, list):
                    for metric, value in feval_ret:
                        result += f"\t{name}-{metric}:{value}"
                else:
                    metric, value = feval_ret
                    result += f"\t{name}-{metric}:{value}"
        return result

    def eval(self, data: DMatrix, name: str = "eval", iteration: int = 0) -> str:
        return self.eval_set([(data, name)], iteration)

    # ---- prediction ------------------------------------------------------------
    def predict(self, data: DMatrix, output_margin: bool = False, pred_leaf: bool = False,
                pred_contribs: bool = False, approx_contribs: bool = False, pred_interactions: bool = False,
                validate_features: bool = True, training: bool = False,
                iteration_range: Tuple[int, int] = (0, 0), strict_shape: bool = False) -> np.ndarray:
        if not isinstance(data, DMatrix):
            raise TypeError("Expecting data to be a DMatrix object")
        # One prediction type at a time (reference core.py:2603-2614): 1 margin,
        # 2 / 3 exact / approximate contributions, 4 / 5 interactions, 6 leaf.
        kinds = [t for flag, t in ((output_margin, 1), (pred_contribs, 3 if approx_contribs else 2),
                                   (pred_interactions, 5 if approx_contribs else 4), (pred_leaf, 6)) if flag]
        if len(kinds) > 1:
            raise ValueError("One type of prediction at a time.")
        config = {"type": kinds[0] if kinds else 0, "training": bool(training),
                  "iteration_begin": int(iteration_range[0]), "iteration_end": int(iteration_range[1]),
                  "strict_shape": bool(strict_shape)}
        shape = ctypes.POINTER(c_bst_ulong)()
        dims = c_bst_ulong()
        result = ctypes.POINTER(ctypes.c_float)()
        _check_call(_LIB.XGBoosterPredictFromDMatrix(self.handle, data.handle, json.dumps(config).encode(),
                                                     ctypes.byref(shape), ctypes.byref(dims), ctypes.byref(result)))
        dims_v = [shape[i] for i in range(dims.value)]
        n = int(np.prod(dims_v)) if dims_v else 0
        out = np.ctypeslib.as_array(result, shape=(n,)).copy() if n else np.zeros(0, np.float32)
        return out.reshape(dims_v)

    def inplace_predict(self, data: Any, iteration_range: Tuple[int, int] = (0, 0), predict_type: str = "value",
                        missing: float = np.nan, validate_features: bool = True, base_margin: Any = None,
                        strict_shape: bool = False) -> np.ndarray:
        """Predict straight from a numpy array, DataFrame or scipy CSR matrix (reference core.py:2642)."""
        if predict_type not in ("value", "margin"):
            raise ValueError(f"predict_type must be 'value' or 'margin', got {predict_type!r}")
        if base_margin is not None:
            dmat = DMatrix(data, base_margin=base_margin, missing=missing)
            return self.predict(dmat, output_margin=predict_type == "margin", iteration_range=iteration_range,
                                strict_shape=strict_shape)
        config = json.dumps({"type": 1 if predict_type == "margin" else 0, "training": False,
                             "iteration_begin": int(iteration_range[0]), "iteration_end": int(iteration_range[1]),
                             "missing": _missing_value(missing), "strict_shape": bool(strict_shape),
                             "cache_id": 0}).encode()
        shape = ctypes.POINTER(c_bst_ulong)()
        dims = c_bst_ulong()
        result = ctypes.POINTER(ctypes.c_float)()
        if type(data).__name__ in ("csc_matrix", "csc_array", "coo_matrix", "coo_array"):
            data = data.tocsr()
        if _is_scipy_csr(data):
            indptr = np.ascontiguousarray(data.indptr, dtype=np.int64)
            indices = np.ascontiguousarray(data.indices, dtype=np.int32)
            values = np.ascontiguousarray(data.data, dtype=np.float32)
            _check_call(_LIB.XGBoosterPredictFromCSR(self.handle, _array_interface(indptr), _array_interface(indices),
                                                     _array_interface(values), c_bst_ulong(data.shape[1]), config,
                                                     None, ctypes.byref(shape), ctypes.byref(dims),
                                                     ctypes.byref(result)))
        else:
            arr = _to_numpy_2d(data)
            _check_call(_LIB.XGBoosterPredictFromDense(self.handle, _array_interface(arr), config, None,
                                                       ctypes.byref(shape), ctypes.byref(dims),
                                                       ctypes.byref(result)))
        dims_v = [shape[i] for i in range(dims.value)]
        n = int(np.prod(dims_v)) if dims_v else 0
        out = np.ctypeslib.as_array(result, shape=(n,)).copy() if n else np.zeros(0, np.float32)
        return out.reshape(dims_v)

    # ---- model inspection ----------------------------------------------------------
    def __getitem__(self, val: Union[int, slice, Any]) -> "Booster":
        """Trees of the rounds in ``val`` as a new Booster (reference core.py:1981)."""
        if isinstance(val, (int, np.integer)) and not isinstance(val, bool):
            val = slice(int(val), int(val) + 1)
        if val is Ellipsis:
            val = slice(0, 0)
        if isinstance(val, tuple):
            raise ValueError("Only supports slicing through 1 dimension.")
        if not isinstance(val, slice):
            raise TypeError(f"Expecting an int, slice or Ellipsis, got {type(val).__name__}")
        start = 0 if val.start is None or val.start is Ellipsis else val.start
        stop = 0 if val.stop is None or val.stop is Ellipsis else val.stop
        if val.stop is not None and val.stop is not Ellipsis and stop < start:
            raise ValueError("Invalid slice", val)
        step = val.step if val.step is not None else 1
        handle = ctypes.c_void_p()
        status = _LIB.XGBoosterSlice(self.handle, ctypes.c_int(start), ctypes.c_int(stop), ctypes.c_int(step),
                                     ctypes.byref(handle))
        if status == -2:
            raise IndexError("Layer index out of range")
        _check_call(status)
        sliced = Booster()
        _check_call(_LIB.XGBoosterFree(sliced.handle))
        sliced.handle = handle
        sliced.feature_names = self.feature_names
        sliced.feature_types = self.feature_types
        return sliced

    def __iter__(self) -> Iterable["Booster"]:
        for i in range(self.num_boosted_rounds()):
            yield self[i]

    def get_dump(self, fmap: Union[str, os.PathLike] = "", with_stats: bool = False,
                 dump_format: str = "text") -> List[str]:
        """One string per tree in the text, JSON or dot format (reference core.py:3198)."""
        fmap = os.fspath(os.path.expanduser(fmap))
        length = c_bst_ulong()
        sarr = ctypes.POINTER(ctypes.c_char_p)()
        _check_call(_LIB.XGBoosterDumpModelEx(self.handle, c_str(fmap), ctypes.c_int(with_stats), c_str(dump_format),
                                              ctypes.byref(length), ctypes.byref(sarr)))
        return [sarr[i].decode() for i in range(length.value)]

    def dump_model(self, fout: Any, fmap: Union[str, os.PathLike] = "", with_stats: bool = False,
                   dump_format: str = "text") -> None:
        """Write the dump to a file or stream (reference core.py:3153)."""
        dumps = self.get_dump(fmap, with_stats, dump_format)
        own = isinstance(fout, (str, os.PathLike))
        f = open(os.fspath(os.path.expanduser(fout)), "w", encoding="utf-8") if own else fout
        try:
            if dump_format == "json":
                f.write("[\n" + ",\n".join(dumps) + "\n]")
            else:
                for i, d in enumerate(dumps):
                    f.write(f"booster[{i}]:\n{d}")
        finally:
            if own:
                f.close()

    def get_score(self, fmap: Union[str, os.PathLike] = "", importance_type: str = "weight") -> Dict[str, float]:
        """Per-feature importance over the split nodes (reference core.py:3250)."""
        fmap = os.fspath(os.path.expanduser(fmap))
        features = ctypes.POINTER(ctypes.c_char_p)()
        scores = ctypes.POINTER(ctypes.c_float)()
        n_features = c_bst_ulong()
        dims = c_bst_ulong()
        shape = ctypes.POINTER(c_bst_ulong)()
        config = json.dumps({"importance_type": importance_type, "feature_map": fmap}).encode()
        _check_call(_LIB.XGBoosterFeatureScore(self.handle, config, ctypes.byref(n_features), ctypes.byref(features),
                                               ctypes.byref(dims), ctypes.byref(shape), ctypes.byref(scores)))
        return {features[i].decode(): float(scores[i]) for i in range(n_features.value)}

    def get_fscore(self, fmap: Union[str, os.PathLike] = "") -> Dict[str, float]:
        return self.get_score(fmap, importance_type="weight")

    # ---- model IO ----------------------------------------------------------------
    def save_model(self, fname: Union[str, os.PathLike]) -> None:
        _check_call(_LIB.XGBoosterSaveModel(self.handle, c_str(os.fspath(fname))))

    def load_model(self, fname: Union[str, os.PathLike, bytearray, bytes]) -> None:
        if isinstance(fname, (bytes, bytearray)):
            buf = (ctypes.c_char * len(fname)).from_buffer_copy(bytes(fname))
            _check_call(_LIB.XGBoosterLoadModelFromBuffer(self.handle, buf, c_bst_ulong(len(fname))))
        else:
            _check_call(_LIB.XGBoosterLoadModel(self.handle, c_str(os.fspath(fname))))

    def save_raw(self, raw_format: str = "ubj") -> bytearray:
        length = c_bst_ulong()
        ptr = ctypes.POINTER(ctypes.c_char)()
        cfg = json.dumps({"format": raw_format}).encode()
        _check_call(_LIB.XGBoosterSaveModelToBuffer(self.handle, cfg, ctypes.byref(length), ctypes.byref(ptr)))
        return bytearray(ctypes.string_at(ptr, length.value))

    def save_config(self) -> str:
        length = c_bst_ulong()
        out = ctypes.c_char_p()
        _check_call(_LIB.XGBoosterSaveJsonConfig(self.handle, ctypes.byref(length), ctypes.byref(out)))
        return out.value.decode()

    def load_config(self, config: str) -> None:
        _check_call(_LIB.XGBoosterLoadJsonConfig(self.handle, config.encode()))

    @property
    def best_iteration(self) -> int:
        """Best round of early stopping, kept as the ``best_iteration`` attribute (reference core.py:3107)."""
        best = self.attr("best_iteration")
        if best is not None:
            return int(best)
        raise AttributeError("`best_iteration` is only defined when early stopping is used.")

    @best_iteration.setter
    def best_iteration(self, iteration: int) -> None:
        self.set_attr(best_iteration=iteration)

    @property
    def best_score(self) -> float:
        best = self.attr("best_score")
        if best is not None:
            return float(best)
        raise AttributeError("`best_score` is only defined when early stopping is used.")

    @best_score.setter
    def best_score(self, score: float) -> None:
        self.set_attr(best_score=score)

    def num_boosted_rounds(self) -> int:
        out = ctypes.c_int()
        _check_call(_LIB.XGBoosterBoostedRounds(self.handle, ctypes.byref(out)))
        return out.value

    def num_features(self) -> int:
        out = c_bst_ulong()
        _check_call(_LIB.XGBoosterGetNumFeature(self.handle, ctypes.byref(out)))
        return out.value

    def profile(self) -> dict:
        out = ctypes.c_char_p()
        _check_call(_LIB.XGBoosterHipProfile(self.handle, ctypes.byref(out)))
        return json.loads(out.value.decode())

    def trees_to_json(self) -> list:
        return json.loads(self.save_raw("json"))["learner"]["gradient_booster"]["model"]["trees"]
