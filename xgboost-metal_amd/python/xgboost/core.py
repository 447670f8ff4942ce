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
from typing import Any, Dict, Iterable, List, Optional, Sequence, Tuple, Union

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


class DMatrix:
    """Data matrix for training and prediction (reference core.py:676)."""

    def __init__(self, data: Any, label: Any = None, *, weight: Any = None, base_margin: Any = None,
                 missing: Optional[float] = None, silent: bool = False, feature_names: Optional[Sequence[str]] = None,
                 feature_types: Optional[Sequence[str]] = None, nthread: Optional[int] = None,
                 enable_categorical: bool = False, **kwargs: Any) -> None:
        self.handle = ctypes.c_void_p()
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

    def __del__(self) -> None:
        if getattr(self, "handle", None) is not None and self.handle.value:
            _check_call(_LIB.XGDMatrixFree(self.handle))
            self.handle = None

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

    def get_quantile_cut(self) -> Tuple[np.ndarray, np.ndarray]:
        """Histogram cut points: (indptr, values) per feature."""
        indptr = ctypes.c_char_p()
        values = ctypes.c_char_p()
        _check_call(_LIB.XGDMatrixGetQuantileCut(self.handle, b"{}", ctypes.byref(indptr), ctypes.byref(values)))
        return _from_interface(indptr.value), _from_interface(values.value)


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
            if key == "eval_metric" and isinstance(val, (list, tuple)):
                val = val[-1] if val else "rmse"
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
        if pred_leaf or pred_contribs or pred_interactions:
            raise XGBoostError("pred_leaf/pred_contribs are not supported by this engine")
        if not isinstance(data, DMatrix):
            raise TypeError("Expecting data to be a DMatrix object")
        config = {"type": 1 if output_margin else 0, "training": bool(training),
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
                        missing: float = np.nan, **kwargs: Any) -> np.ndarray:
        dmat = DMatrix(data, missing=missing)
        return self.predict(dmat, output_margin=predict_type == "margin", iteration_range=iteration_range)

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
