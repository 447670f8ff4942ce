"""BASELINE configs 3 and 4 at their full sizes, through properties that do
not depend on the oracle finishing (it would take hours there):

- every code path that must not change the result trains the same trees:
  the stable and the atomic-claim partition, the subsample's compacted row
  list and the full one (C4), the CSR root histogram from the column-major
  copy and from device atomics (C3);
- the training margins the partition kernels accumulate (the prediction
  cache) equal a fresh prediction that walks the trees, bit for bit;
- the quantile cuts are strictly increasing per feature, and every split
  threshold is one of its feature's cuts; config 4's 10M x 128 cuts also
  equal the CPU oracle's bit for bit.

Config 2 at full size is pinned by the reference's published prediction
hash (test_gpu_parity.py::test_published_prediction_hashes) and the oracle;
the quantile sketch beyond 2^24 entries a feature (where integer weight sums
stop being exact) is checked against the oracle."""
import json

import numpy as np
import pytest
import scipy.sparse as sp

import workloads as W

pytestmark = pytest.mark.gpu


def _trees(bst):
    return json.loads(bst.save_raw("json"))["learner"]["gradient_booster"]["model"]["trees"]


def _margins_equal_walk(xgb, bst, d, fresh):
    np.testing.assert_array_equal(bst.predict(d, output_margin=True).view(np.uint32),
                                  bst.predict(fresh, output_margin=True).view(np.uint32))


@pytest.fixture(scope="module")
def config4_data():
    return W.config4()


def test_config4_full_size_paths_agree(xgb, config4_data):
    X, y = config4_data
    d = xgb.DMatrix(X, label=y)
    params = dict(W.CONFIG_PARAMS[4], seed=7)
    base = xgb.train(params, d, 3)
    variant = xgb.train(dict(params, hip_stable_partition=0, hip_compact_sampled=0), d, 3)
    trees = _trees(base)
    assert trees == _trees(variant)
    # A real depth-10 tree with 1024-bin thresholds.
    assert max(len(t["split_indices"]) for t in trees) > 1000
    fresh = xgb.DMatrix(X[:2_000_000])
    np.testing.assert_array_equal(
        base.predict(d, output_margin=True)[:2_000_000].view(np.uint32),
        base.predict(fresh, output_margin=True).view(np.uint32))


def test_config4_full_size_cuts(xgb, config4_data):
    """The sketch's cuts at 10M rows and 1024 bins equal the CPU oracle's bit
    for bit for all 128 features (the oracle sketches one feature per
    thread); and by properties: strictly increasing per feature, at most
    max_bin of them, the integer columns' cuts at most one per distinct value
    (1,000), and every split threshold of a tree one of its feature's cuts."""
    import oracle_lib as O
    X, y = config4_data
    d = xgb.DMatrix(X, label=y)
    bst = xgb.train(dict(W.CONFIG_PARAMS[4], seed=7), d, 1)
    indptr, values = d.get_quantile_cut()
    assert len(indptr) == 129
    ocuts, ocounts, _ = O.sketch_cuts(X, 1024)
    np.testing.assert_array_equal(np.diff(indptr), ocounts)
    for f in range(128):
        np.testing.assert_array_equal(values[indptr[f]:indptr[f + 1]].view(np.uint32),
                                      ocuts[f, :ocounts[f]].view(np.uint32), err_msg=f"feature {f}")
    for f in range(128):
        cuts = values[indptr[f]:indptr[f + 1]]
        assert 2 <= len(cuts) <= 1024
        assert np.all(np.diff(cuts) > 0)
        if f >= 96:
            assert len(cuts) <= 1001
    for t in _trees(bst):
        for f, thr, left in zip(t["split_indices"], t["split_conditions"], t["left_children"]):
            if left >= 0:
                assert np.float32(thr) in values[indptr[f]:indptr[f + 1]]


def test_config3_full_size_paths_agree(xgb):
    indptr, indices, values, y = W.config3()
    csr = sp.csr_matrix((values, indices, indptr), shape=(len(indptr) - 1, 2000))
    d = xgb.DMatrix(csr, label=y)
    params = dict(W.CONFIG_PARAMS[3])
    base = xgb.train(params, d, 3)
    variant = xgb.train(dict(params, hip_stable_partition=0, hip_csr_root_columns=0), d, 3)
    assert _trees(base) == _trees(variant)
    fresh = xgb.DMatrix(csr[:200_000])
    np.testing.assert_array_equal(base.predict(d, output_margin=True)[:200_000].view(np.uint32),
                                  base.predict(fresh, output_margin=True).view(np.uint32))


def test_config2_full_size_matches_oracle(xgb):
    """BASELINE config 2's own generator at its full 262,144 x 64, depth 8,
    against the CPU oracle: the margins after 10 rounds bit for bit (the
    bench compares the full 100-round fit's predictions the same way)."""
    import os

    import oracle_lib as O
    X, y = W.config2()
    bst = xgb.train(dict(W.CONFIG_PARAMS[2]), xgb.DMatrix(X, label=y), 10)
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    ref = O.train(X, y, O.make_params(max_depth=8, max_bin=256, eta=0.3, nthread=threads), 10)
    got = bst.predict(xgb.DMatrix(X), output_margin=True)
    np.testing.assert_array_equal(got.view(np.uint32), ref["margin"].view(np.uint32))


def test_sketch_beyond_exact_integer_sums():
    """Unweighted features with more than 2^24 entries leave the exact path:
    their batches are sorted as runs carrying their lengths and summarized with
    serial binary32 sums (the weighted path's rules). One continuous feature
    and one of 64-row runs over 50 values, against the oracle bit for bit."""
    import device_lib as D
    import oracle_lib as O
    n = (1 << 24) + 200000
    rng = np.random.default_rng(7)
    X = np.empty((n, 2), np.float32)
    X[:, 0] = rng.normal(size=n).astype(np.float32)
    X[:, 1] = np.repeat(rng.integers(0, 50, size=n // 64 + 1), 64)[:n].astype(np.float32)
    cuts, counts = D.sketch_cuts(X, 256)
    ocuts, ocounts, _ = O.sketch_cuts(X, 256)
    np.testing.assert_array_equal(counts, ocounts)
    for f in range(X.shape[1]):
        np.testing.assert_array_equal(cuts[f, :counts[f]].view(np.uint32), ocuts[f, :counts[f]].view(np.uint32))
