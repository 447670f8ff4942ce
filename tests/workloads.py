"""Synthetic workloads: BASELINE.json's configs and the reference's published
known-answer workloads (benchmarks/controlled_comparison.py:68-72 of the
reference: seed 1337, y = 2*x0 + x1^2 + 0.1*N)."""
import numpy as np

# Prediction SHA-256 known answers published by the reference for stock
# XGBoost 3.4.1 CPU hist (identical on three machines), with their inputs.
KNOWN_ANSWERS = {
    "dense100": dict(rows=100000, features=32, depth=6,
                     input_sha256="1dfa73f3445387c17a823cf2c0567d2275520de6c98d1ab17caf3a529a9c06ef",
                     label_sha256="74b851f7b4111a68421f0f2e9d00b147ec9afb1eab07caeb0298bef9aa17903c",
                     prediction_sha256="c891e08b2e9a517abd616551e4938b1eea1b4ffc1f34c77f127e3cee238fe371",
                     rmse=0.1233987458001251),
    "dense262": dict(rows=262144, features=64, depth=8,
                     prediction_sha256="0497a073f27cad24af247bc28a49e0f5d9423d8dacac6577b89bbca169696a5a",
                     rmse=0.10546882076795792),
    "missing100": dict(rows=100000, features=32, depth=6,
                       prediction_sha256="8e7bf89a1af7dc99661b3a0681fbc8ad1d2a25ae749538a587191f381588e973",
                       rmse=0.7557960928611526),
}
KNOWN_PARAMS = {"objective": "reg:squarederror", "tree_method": "hist", "max_bin": 256, "eta": 0.3, "seed": 42}


def known_answer_data(case):
    spec = KNOWN_ANSWERS[case]
    rng = np.random.default_rng(1337)
    X = rng.normal(size=(spec["rows"], spec["features"])).astype(np.float32)
    y = (2 * X[:, 0] + X[:, 1] ** 2 + 0.1 * rng.normal(size=spec["rows"])).astype(np.float32)
    if case == "missing100":
        X[rng.random(X.shape) < 0.15] = np.nan
    return X, y


def config0(rows=100000, cols=32, seed=1337):
    """dense regression, y = X.w + 0.1 N."""
    rng = np.random.default_rng(seed)
    X = rng.normal(size=(rows, cols)).astype(np.float32)
    w = rng.normal(size=cols).astype(np.float32)
    y = (X @ w + 0.1 * rng.normal(size=rows)).astype(np.float32)
    return X, y


def config1(rows=100000, cols=32, seed=1337):
    """config 0 with 15% of entries set to NaN after the label."""
    rng = np.random.default_rng(seed)
    X = rng.normal(size=(rows, cols)).astype(np.float32)
    w = rng.normal(size=cols).astype(np.float32)
    y = (X @ w + 0.1 * rng.normal(size=rows)).astype(np.float32)
    X[rng.random(X.shape) < 0.15] = np.nan
    return X, y


def config2(rows=262144, cols=64, seed=1337):
    """BASELINE config 2 (north star): y = X.w + 0.5 sin(x0 x1) + 0.1 N."""
    rng = np.random.default_rng(seed)
    X = rng.normal(size=(rows, cols)).astype(np.float32)
    w = rng.normal(size=cols).astype(np.float32)
    y = (X @ w + 0.5 * np.sin(X[:, 0] * X[:, 1]) + 0.1 * rng.normal(size=rows)).astype(np.float32)
    return X, y


CONFIG_PARAMS = {
    0: {"objective": "reg:squarederror", "tree_method": "hist", "max_depth": 6, "max_bin": 256, "eta": 0.3,
        "lambda": 1, "min_child_weight": 1},
    1: {"objective": "reg:squarederror", "tree_method": "hist", "max_depth": 6, "max_bin": 256, "eta": 0.3,
        "lambda": 1, "min_child_weight": 1},
    2: {"objective": "reg:squarederror", "tree_method": "hist", "max_depth": 8, "max_bin": 256, "eta": 0.3,
        "lambda": 1},
}
