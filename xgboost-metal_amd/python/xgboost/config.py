"""Global configuration (the reference's python-package/xgboost/config.py
surface: set_config, get_config, config_context) over the library's
thread-local XGBSetGlobalConfig / XGBGetGlobalConfig.

Keys: verbosity, use_rmm, nthread (accepted, as upstream), and std_shuffle
("libstdc++" or "libc++"): the standard library whose std::shuffle draws the
rows of xgb.cv's folds."""
import contextlib
import ctypes
import json
from typing import Any, Dict, Iterator

from .core import _LIB, _check_call


def set_config(**new_config: Any) -> None:
    """Set global configuration keys for the calling thread."""
    _check_call(_LIB.XGBSetGlobalConfig(json.dumps(new_config).encode()))


def get_config() -> Dict[str, Any]:
    """The calling thread's global configuration."""
    out = ctypes.c_char_p()
    _check_call(_LIB.XGBGetGlobalConfig(ctypes.byref(out)))
    return json.loads(out.value.decode())


@contextlib.contextmanager
def config_context(**new_config: Any) -> Iterator[None]:
    """Apply `new_config` inside the block and restore the previous values."""
    previous = get_config()
    set_config(**new_config)
    try:
        yield
    finally:
        restore = {key: previous[key] for key in new_config if key in previous}
        if restore:
            set_config(**restore)
