"""CPU-side checks of the C-ABI library: it loads, exports every symbol that
include/mk.h declares, and its host-side index builder matches the oracle
bit-exactly.  No device calls."""
import ctypes as C
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
    assert L.mk_abi_version() == capi.ABI_VERSION == 7


_STRUCTS = {"mk_gemm_args": capi.GemmArgs, "mk_gemm_ar_args": capi.GemmArArgs, "mk_gemm_ar2_args": capi.GemmAr2Args, "mk_ag_gemm_args": capi.AgGemmArgs, "mk_gemm_rs_args": capi.GemmRsArgs,
            "mk_moe_index": capi.MoeIndex, "mk_moe_permute_args": capi.MoePermuteArgs,
            "mk_moe_grouped_gemm_args": capi.MoeGroupedGemmArgs, "mk_moe_combine_args": capi.MoeCombineArgs,
            "mk_moe_ffn_args": capi.MoeFfnArgs, "mk_moe_index_dev_args": capi.MoeIndexDevArgs}


def test_struct_layouts_match_header(tmp_path):
    """Every ctypes struct has the size and field offsets the C compiler gives
    the header's struct (compiled with the host gcc)."""
    import shutil
    import subprocess
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no host C compiler")
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{ROOT / "include" / "mk.h"}"', "int main(void) {"]
    for cname, cls in _STRUCTS.items():
        lines.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for f, _ in cls._fields_:
            lines.append(f'  printf("{cname} {f} %zu\\n", offsetof({cname}, {f}));')
    lines.append("  return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run([cc, str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = {tuple(l.split()[:2]): int(l.split()[2]) for l in out if l}
    for cname, cls in _STRUCTS.items():
        assert got[(cname, "size")] == C.sizeof(cls), cname
        for f, _ in cls._fields_:
            assert got[(cname, f)] == getattr(cls, f).offset, (cname, f)


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


_ARGS_ENTRIES = {"mk_gemm": capi.GemmArgs, "mk_ag_gemm": capi.AgGemmArgs, "mk_ag_gemm_noalloc": capi.AgGemmArgs,
                 "mk_gemm_rs": capi.GemmRsArgs, "mk_gemm_ar": capi.GemmArArgs, "mk_gemm_ar_two_shot": capi.GemmAr2Args,
                 "mk_moe_permute": capi.MoePermuteArgs, "mk_moe_grouped_gemm": capi.MoeGroupedGemmArgs,
                 "mk_moe_combine": capi.MoeCombineArgs, "mk_moe_ffn_combine": capi.MoeFfnArgs,
                 "mk_moe_build_indices_dev": capi.MoeIndexDevArgs}


@pytest.mark.parametrize("name", sorted(_ARGS_ENTRIES))
def test_entry_points_refuse_missing_arguments(name):
    """Every args-struct entry point refuses a NULL struct (a negative code,
    i.e. an argument error and not a HIP error, with a message naming the
    entry point) and a zero-filled struct (NULL operands, zero sizes), both
    before touching a device: this container has none, so any device call
    would return a positive HIP error instead."""
    L = capi.lib()
    L.mk_last_error_string.restype = C.c_char_p
    fn = getattr(L, name)
    assert fn(None, None) < 0
    assert name.encode() in L.mk_last_error_string()
    empty = _ARGS_ENTRIES[name]()  # every pointer NULL, every size 0
    assert fn(C.byref(empty), None) < 0, L.mk_last_error_string()
