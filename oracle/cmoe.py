"""ctypes wrapper of oracle/moe_index.c (test-only).  Builds it on first use."""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
SO = HERE / "_build" / "liboracle_moe.so"


def _lib():
    if not SO.exists():
        subprocess.run(["make", "-C", str(HERE)], check=True, capture_output=True)
    L = C.CDLL(str(SO))
    L.oracle_moe_sizes.restype = C.c_int
    L.oracle_moe_build.restype = C.c_int
    return L


def build_indices_c(topk_ids: np.ndarray, gates: np.ndarray, e0: int, n_local: int, row_block: int = 128) -> dict:
    ids = np.ascontiguousarray(topk_ids, dtype=np.int32)
    g = np.ascontiguousarray(gates, dtype=np.float32)
    T, k = ids.shape
    L = _lib()
    R, Rp = C.c_int64(), C.c_int64()
    p = lambda a: a.ctypes.data_as(C.c_void_p)
    assert L.oracle_moe_sizes(p(ids), T, k, e0, n_local, row_block, C.byref(R), C.byref(Rp)) == 0
    R, Rp = R.value, Rp.value
    out = {
        "padded_tokens_per_expert": np.zeros(n_local, np.int32),
        "pull_indices": np.zeros((Rp, 3), np.int32),
        "row_expert": np.zeros(Rp, np.int32),
        "row_weight": np.zeros(Rp, np.float32),
        "owner_offset": np.zeros(T + 1, np.int32),
        "row_to_slot": np.zeros(Rp, np.int32),
        "row_to_owner": np.zeros(Rp, np.int32),
        "slot_to_row": np.zeros(max(R, 1), np.int32),
    }
    o = out
    assert L.oracle_moe_build(p(ids), p(g), T, k, e0, n_local, row_block, p(o["padded_tokens_per_expert"]),
                              p(o["pull_indices"]), p(o["row_expert"]), p(o["row_weight"]), p(o["owner_offset"]),
                              p(o["row_to_slot"]), p(o["row_to_owner"]), p(o["slot_to_row"])) == 0
    out["slot_to_row"] = out["slot_to_row"][:R]
    out["R"], out["R_pad"] = R, Rp
    return out
