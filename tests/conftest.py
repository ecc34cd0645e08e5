import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "forge-db_amd"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C ABI)")


def tie_aware_match(ids_a, d_a, ids_b, d_b, rel=1e-4):
    """True when two ascending top-k lists agree up to ties: every id outside
    the intersection sits at a distance within `rel` of the k-th distance of
    the list it comes from, and the distance vectors agree within `rel`."""
    ids_a, ids_b = list(map(int, ids_a)), list(map(int, ids_b))
    if len(ids_a) != len(ids_b):
        return False, f"lengths {len(ids_a)} != {len(ids_b)}"
    if not ids_a:
        return True, ""
    da, db = np.asarray(d_a, np.float64), np.asarray(d_b, np.float64)
    scale = np.maximum(np.abs(db), 1e-30)
    if np.any(np.abs(da - db) > rel * scale + 1e-30):
        return False, f"distances differ: {da} vs {db}"
    sa, sb = set(ids_a), set(ids_b)
    kth = max(abs(da[-1]), abs(db[-1]))
    for i, x in enumerate(ids_a):
        if x not in sb and abs(da[i] - db[-1]) > rel * max(kth, 1e-30):
            return False, f"id {x} (d={da[i]}) missing from the other list, kth={db[-1]}"
    for i, x in enumerate(ids_b):
        if x not in sa and abs(db[i] - da[-1]) > rel * max(kth, 1e-30):
            return False, f"id {x} (d={db[i]}) missing from the first list, kth={da[-1]}"
    return True, ""


@pytest.fixture(scope="session")
def small_ivfpq():
    """A small IVF-PQ index trained by the oracle on the integer-mixture
    workload (20k x 128, nlist 64, M 16) plus 64 queries."""
    import refcpu
    from forgedb import datagen
    base, queries = datagen.workload("ivfpq_int", n=20_000, nq=64)
    ix = refcpu.IvfPq.build(base, nlist=64, M=16, seed=7)
    return dict(base=base, queries=queries, oracle=ix, art=ix.export())
