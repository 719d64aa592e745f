"""CPU-side checks of the C-ABI library: it loads, exports every symbol that
include/mk.h declares, and its host-side index builder matches the oracle
bit-exactly.  No device calls."""
import re
from pathlib import Path

import numpy as np
import pytest

from mkernel_amd import capi, ops, workloads as wl
from oracle import moe as om
from oracle.cmoe import build_indices_c

ROOT = Path(__file__).resolve().parent.parent


def _header_symbols():
    text = (ROOT / "include" / "mk.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int32_t|int64_t|const char\*)\s+(mk_\w+)\s*\(", text, re.M)))


def test_header_and_binding_agree():
    assert _header_symbols() == sorted(capi.EXPORTS)


def test_library_exports_every_declared_symbol():
    L = capi.lib()
    for name in _header_symbols():
        assert hasattr(L, name), name
    assert L.mk_abi_version() == 1


@pytest.mark.parametrize("cls,nfields", [(capi.GemmArgs, 12), (capi.AgGemmArgs, 16), (capi.GemmRsArgs, 20),
                                         (capi.MoeIndex, 11), (capi.MoeGroupedGemmArgs, 12)])
def test_struct_layouts(cls, nfields):
    assert len(cls._fields_) == nfields


def test_index_builder_matches_oracle_tiny():
    import json
    g = json.loads((ROOT / "tests" / "golden" / "index_tiny.json").read_text())
    o = ops.moe_build_indices(np.array(g["topk_ids"]), np.array(g["gates"], np.float32), g["e0"], g["n_local"],
                              g["row_block"])
    for key, val in g["expected"].items():
        got = o[key].tolist()
        if key == "row_weight":
            assert np.allclose(got, val)
        else:
            assert got == val, key


@pytest.mark.parametrize("T,rank", [(256, 0), (4096, 0), (4096, 5)])
def test_index_builder_matches_oracle(T, rank):
    cfg = wl.MoeCfg(tokens=T, rank=rank)
    ids, gates = wl.zipf_routing(T, cfg.experts, cfg.topk, cfg.zipf_s, 6)
    lib_o = ops.moe_build_indices(ids, gates, cfg.e0, cfg.n_local)
    ref = om.build_indices_np(ids, gates, cfg.e0, cfg.n_local)
    cref = build_indices_c(ids, gates, cfg.e0, cfg.n_local)
    for key in ("padded_tokens_per_expert", "local_rb_per_expert", "pull_indices", "row_expert", "rb_expert", "rb_rows",
                "row_weight", "owner_offset", "row_to_slot", "row_to_owner", "slot_to_row"):
        assert np.array_equal(lib_o[key], ref[key]), key
        if key in cref:
            assert np.array_equal(lib_o[key], cref[key]), key
    assert lib_o["R"] == ref["R"] and lib_o["R_pad"] == ref["R_pad"]


def test_index_builder_rejects_bad_args():
    with pytest.raises(capi.MkError):
        ops.moe_build_indices(np.zeros((4, 2), np.int32), np.zeros((4, 2), np.float32), 0, 0)
