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


def config3(rows=1_000_000, cols=2000, nnz=20, informative=200, seed=1337):
    """CSR classification.  Per row `nnz` distinct columns
    drawn uniformly (24 draws a row, the first `nnz` distinct ones in draw
    order; rows with fewer are drawn again), sorted; values lognormal(0, 1);
    w ~ N(0, sd 0.25) on `informative` random columns; y ~ Bernoulli(sigmoid(
    sum v w)).  Draw order: columns, values, informative columns, their
    weights, labels.  Returns (indptr int64, indices int32, values float32,
    labels float32)."""
    rng = np.random.default_rng(seed)
    idx = np.empty((rows, nnz), np.int64)
    todo = np.arange(rows)
    while len(todo):
        draw = rng.integers(0, cols, size=(len(todo), 24))
        order = np.argsort(draw, axis=1, kind="stable")
        srt = np.take_along_axis(draw, order, axis=1)
        dup_sorted = np.zeros_like(srt, dtype=bool)
        dup_sorted[:, 1:] = srt[:, 1:] == srt[:, :-1]
        dup = np.empty_like(dup_sorted)
        np.put_along_axis(dup, order, dup_sorted, axis=1)
        keep = ~dup & (np.cumsum(~dup, axis=1) <= nnz)
        ok = keep.sum(axis=1) == nnz
        idx[todo[ok]] = draw[ok][keep[ok]].reshape(-1, nnz)
        todo = todo[~ok]
    idx.sort(axis=1)
    values = rng.lognormal(0.0, 1.0, size=(rows, nnz)).astype(np.float32)
    wcols = rng.choice(cols, size=informative, replace=False)
    w = np.zeros(cols, np.float32)
    w[wcols] = rng.normal(0.0, 0.25, size=informative).astype(np.float32)
    s = (values * w[idx]).sum(axis=1)
    y = (rng.random(rows) < 1.0 / (1.0 + np.exp(-s))).astype(np.float32)
    indptr = np.arange(0, (rows + 1) * nnz, nnz, dtype=np.int64)
    return indptr, idx.reshape(-1).astype(np.int32), values.reshape(-1), y


def weighted_million():
    """The reference's weighted dense-root construction
    (tests/test_scalar_root_statistics.py:66-80): 1,000,000 rows of
    default_rng(43) N(0,1) x 64, y = 2 x0 + x1^2 + N(0, 0.1), the first four
    columns kept; weights default_rng(144) uniform(0.1, 2).  With depth 1,
    256 bins and seed 9, one round's root base weight has the bits
    2915099116 in the reference's CPU oracle build."""
    rng = np.random.default_rng(43)
    original = rng.normal(size=(1000000, 64)).astype(np.float32)
    noise = rng.normal(0, 0.1, len(original))
    y = (2 * original[:, 0] + original[:, 1] ** 2 + noise).astype(np.float32)
    X = original[:, :4].copy()
    del original
    weight = np.random.default_rng(144).uniform(0.1, 2, len(X)).astype(np.float32)
    return X, y, weight


WEIGHTED_MILLION_ROOT_BITS = 2915099116


def weighted_benchmark():
    """The reference's 4096-bin construction (tests/test_parent_statistics.py:
    55-68): 100,000 rows of default_rng(43) N(0,1) x 32, y = 2 x0 + x1^2 +
    N(0, 0.1), the first four columns kept; weights default_rng(144)
    uniform(0.1, 2).  With depth 1, max_bin 4096 and seed 9, one round's root
    base weight has the bits 2990026907 in the reference's CPU oracle build."""
    rng = np.random.default_rng(43)
    original = rng.normal(size=(100000, 32)).astype(np.float32)
    noise = rng.normal(0, 0.1, len(original))
    y = (2 * original[:, 0] + original[:, 1] ** 2 + noise).astype(np.float32)
    X = original[:, :4].copy()
    weight = np.random.default_rng(144).uniform(0.1, 2.0, len(X)).astype(np.float32)
    return X, y, weight


WEIGHTED_BENCHMARK_ROOT_BITS = 2990026907
WEIGHTED_BENCHMARK_PARAMS = {"tree_method": "hist", "max_depth": 1, "max_bin": 4096, "seed": 9}
WEIGHTED_MILLION_PARAMS = {"tree_method": "hist", "max_depth": 1, "max_bin": 256, "seed": 9}


def config4(rows=10_000_000, seed=1337, chunk=1 << 20):
    """columns 0-63 N(0,1), 64-95 U(0,1), 96-127 integers in
    [0, 999] as float32; y ~ Bernoulli(sigmoid(X[:, :16] . w + 0.3 N)).  Drawn
    in row chunks (float32 storage) so the float64 temporaries stay small."""
    rng = np.random.default_rng(seed)
    w = rng.normal(size=16)
    X = np.empty((rows, 128), np.float32)
    y = np.empty(rows, np.float32)
    for a in range(0, rows, chunk):
        b = min(rows, a + chunk)
        n = b - a
        X[a:b, :64] = rng.normal(size=(n, 64))
        X[a:b, 64:96] = rng.random((n, 32))
        X[a:b, 96:] = rng.integers(0, 1000, size=(n, 32))
        s = X[a:b, :16].astype(np.float64) @ w + 0.3 * rng.normal(size=n)
        y[a:b] = rng.random(n) < 1.0 / (1.0 + np.exp(-s))
    return X, y


def csr_to_dense(indptr, indices, values, cols):
    """The dense matrix of a CSR matrix, NaN at the absent entries."""
    rows = len(indptr) - 1
    X = np.full((rows, cols), np.nan, np.float32)
    r = np.repeat(np.arange(rows), np.diff(indptr))
    X[r, indices] = values
    return X


CONFIG_PARAMS = {
    0: {"objective": "reg:squarederror", "tree_method": "hist", "max_depth": 6, "max_bin": 256, "eta": 0.3,
        "lambda": 1, "min_child_weight": 1},
    1: {"objective": "reg:squarederror", "tree_method": "hist", "max_depth": 6, "max_bin": 256, "eta": 0.3,
        "lambda": 1, "min_child_weight": 1},
    2: {"objective": "reg:squarederror", "tree_method": "hist", "max_depth": 8, "max_bin": 256, "eta": 0.3,
        "lambda": 1},
    3: {"objective": "binary:logistic", "tree_method": "hist", "max_depth": 8, "max_bin": 256, "eta": 0.1},
    4: {"objective": "binary:logistic", "tree_method": "hist", "max_depth": 10, "max_bin": 1024, "eta": 0.1,
        "subsample": 0.8, "colsample_bytree": 0.8},
}
