"""Packing of paged_attention's request dicts (native extension vs numpy).

Both implementations must give the same int32 tables / lengths /
shared-prefix statement and raise the same errors, under the reference's
rules (kernels/paged_attention.py:36-48): n_blocks = min(len(blocks),
ceil(seq_len / bs)), length cut to the table, ids outside [-NB, NB) raise
IndexError, negative ids count from the end, no blocks raises RuntimeError.
The shared-prefix lengths are checked against cf_hip.ops.shared_prefix_lens.
"""

from __future__ import annotations

import random

import numpy as np
import pytest

from cf_hip import ops
from kernels import paged_attention as pa

native = pytest.mark.skipif(pa._pack_native is None, reason="_tablepack extension not built")


def _both(bt, sl, bs, nb):
    width = max(len(t) for t in bt.values())
    outs = []
    for fn in (pa._pack_native, pa._pack_tables_py):
        buf = np.full(len(bt) * (width + 2), -7, dtype=np.int32)
        mb = fn(bt, sl, bs, nb, buf, width)
        n = len(bt)
        outs.append((mb, buf[: n * mb].reshape(n, mb).copy(), buf[n * mb: n * (mb + 1)].copy(),
                     buf[n * (mb + 1): n * (mb + 2)].copy()))
    return outs


@native
@pytest.mark.parametrize("seed", range(10))
def test_native_equals_numpy(seed):
    rng = random.Random(seed)
    nb, bs = 500, rng.choice([8, 16, 32])
    prefix = [rng.randrange(-nb, nb) for _ in range(rng.randint(0, 12))]
    bt, sl = {}, {}
    for r in range(rng.randint(1, 40)):
        t = (prefix if rng.random() < 0.5 else []) + [rng.randrange(-nb, nb) for _ in range(rng.randint(1, 30))]
        kind = rng.random()
        rid = f"r{r}" if rng.random() < 0.8 else r  # ids need not be strings
        bt[rid] = t if kind < 0.6 else (tuple(t) if kind < 0.8 else np.asarray(t))
        if rng.random() < 0.8:
            sl[rid] = rng.randint(1, len(t) * bs + 40)
    (m1, t1, l1, s1), (m2, t2, l2, s2) = _both(bt, sl, bs, nb)
    assert m1 == m2
    np.testing.assert_array_equal(t1, t2)
    np.testing.assert_array_equal(l1, l2)
    np.testing.assert_array_equal(s1, s2)
    # the shared-prefix statement is the helper's on the used (wrapped) tables
    used = [list(t1[i][: -(-int(l1[i]) // bs)]) for i in range(len(bt))]
    assert list(s1) == ops.shared_prefix_lens(used, list(l1), bs)


@native
def test_known_answer():
    bt = {"a": [3, -1, 4], "b": [3, 9], "c": [5]}
    sl = {"a": 40, "b": 17}
    (mb, t, l, s), _ = _both(bt, sl, 16, 10)
    assert mb == 3
    np.testing.assert_array_equal(t, [[3, 9, 4], [3, 9, 0], [5, 0, 0]])
    np.testing.assert_array_equal(l, [40, 17, 16])
    np.testing.assert_array_equal(s, [0, 17, 0])


@native
@pytest.mark.parametrize("fn", ["native", "numpy"])
def test_errors(fn):
    f = pa._pack_native if fn == "native" else pa._pack_tables_py
    buf = np.zeros(64, dtype=np.int32)
    with pytest.raises(IndexError, match="out of range"):
        f({"a": [1, 10]}, {}, 16, 10, buf, 2)
    with pytest.raises(IndexError, match="out of range"):
        f({"a": [-11]}, {}, 16, 10, buf, 1)
    with pytest.raises(RuntimeError, match="no KV blocks"):
        f({"a": [1]}, {"a": 0}, 16, 10, buf, 1)
    with pytest.raises(RuntimeError, match="no KV blocks"):
        f({"a": []}, {}, 16, 10, buf, 1)
    # an id past the length is never read, so it is not checked
    assert f({"a": [1, 99]}, {"a": 16}, 16, 10, buf, 2) == 1


def test_width_matches_python():
    from cf_hip._tablepack import width

    tables = {"a": [1, 2, 3], "b": [], "c": list(range(40)), "d": (5, 6)}
    assert width(tables) == max(len(t) for t in tables.values()) == 40
    assert width({}) == 0
    with pytest.raises(TypeError):
        width([[1, 2]])
