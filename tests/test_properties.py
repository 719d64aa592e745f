"""Property-based checks (hypothesis) of the host index builder against the
oracle's restatements of the reference's Python builders, over random
routings: token counts (including 0 and 1), top-k widths, duplicate experts
inside a token, experts outside the local range, and row-block sizes."""
import numpy as np
import pytest
from hypothesis import HealthCheck, given, settings, strategies as st

from mkernel_amd import ops
from oracle import moe as om

TABLES = ("padded_tokens_per_expert", "local_rb_per_expert", "pull_indices", "row_expert", "rb_expert", "rb_rows",
          "row_weight", "owner_offset", "row_to_slot", "row_to_owner", "slot_to_row")


@st.composite
def routings(draw):
    T = draw(st.integers(0, 70))
    k = draw(st.integers(1, 9))
    E = draw(st.integers(1, 40))
    n_local = draw(st.integers(1, E))
    e0 = draw(st.integers(0, E - n_local))
    row_block = draw(st.sampled_from([1, 2, 8, 128]))
    seed = draw(st.integers(0, 2 ** 31 - 1))
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, E, size=(T, k)).astype(np.int32)  # duplicates inside a token allowed
    gates = rng.random((T, k), dtype=np.float32)
    return ids, gates, e0, n_local, row_block


@settings(max_examples=150, deadline=None, suppress_health_check=[HealthCheck.too_slow])
@given(routings())
def test_host_builder_matches_python_oracle(r):
    ids, gates, e0, n_local, row_block = r
    host = ops.moe_build_indices(ids, gates, e0, n_local, row_block)
    ref = om.build_indices_py(ids.tolist(), gates.tolist(), e0, n_local, row_block)
    for f in TABLES:
        h = np.asarray(host[f])
        o = np.asarray(ref[f], dtype=h.dtype).reshape(h.shape)
        if h.dtype == np.float32:
            assert np.array_equal(h.view(np.uint32), o.view(np.uint32)), f
        else:
            assert np.array_equal(h, o), f
    R = sum(1 for t in range(ids.shape[0]) for e in ids[t] if e0 <= e < e0 + n_local)
    assert host["R"] == R
    assert host["R_pad"] % row_block == 0 and host["R_pad"] >= R
