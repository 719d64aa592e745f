"""ctypes binding of libmk's C-ABI (include/mk.h).

This is the only Python module that touches the shared library.  Structures
mirror include/mk.h field by field; every call checks the return code and
raises :class:`MkError` with ``mk_last_error_string()``.  There is no fallback
path: if libmk.so is missing, loading raises.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libmk.so"

ROW_BLOCK = 128
ABI_VERSION = 7  # include/mk.h mk_abi_version(): the structures below match this layout

EXPORTS = (
    "mk_gemm",
    "mk_ag_gemm",
    "mk_ag_gemm_noalloc",
    "mk_ag_gemm_noalloc_scratch_bytes",
    "mk_gemm_rs",
    "mk_gemm_ar",
    "mk_gemm_ar_two_shot",
    "mk_moe_index_sizes",
    "mk_moe_build_indices",
    "mk_moe_index_workspace_bytes",
    "mk_moe_build_indices_dev",
    "mk_moe_permute",
    "mk_moe_grouped_gemm",
    "mk_moe_combine",
    "mk_moe_invert_slots",
    "mk_moe_tile_rows",
    "mk_moe_ffn_combine",
    "mk_query_workspace_bytes",
    "mk_probe_mfma_ceiling",
    "mk_probe_threads",
    "mk_device_cu_count",
    "mk_last_error_string",
    "mk_abi_version",
    "mk_epoch_advance",
)

vp = C.c_void_p
i64 = C.c_int64
i32 = C.c_int32
u32 = C.c_uint32


class MkError(RuntimeError):
    """Non-zero return from libmk (negative: argument/shape, positive: HIP)."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed ({code}): {msg}")
        self.code = code


class GemmArgs(C.Structure):
    _fields_ = [("A", vp), ("B", vp), ("C", vp), ("M", i64), ("N", i64), ("K", i64),
                ("lda", i64), ("ldb", i64), ("ldc", i64), ("num_cus", i32), ("tile_m", i32),
                ("waves", i32), ("split_ws", vp), ("split_ws_bytes", i64)]


class AgGemmArgs(C.Structure):
    _fields_ = [("A_shards", vp), ("A_full", vp), ("B", vp), ("C", vp),
                ("M", i64), ("N", i64), ("K", i64),
                ("flags", vp), ("stage_order", vp), ("epoch", u32), ("gated", i32),
                ("num_producers", i32), ("num_cus", i32), ("spin_limit", u32), ("error_word", vp),
                ("stage_counters", vp), ("split_ws", vp), ("split_ws_bytes", i64), ("epoch_ptr", vp),
                ("n_present", i32)]


class GemmRsArgs(C.Structure):
    _fields_ = [("A", vp), ("B", vp), ("workspace", vp), ("output", vp), ("peer_src", vp),
                ("peer_recv", vp), ("M", i64), ("N", i64), ("K", i64), ("world", i32), ("rank", i32),
                ("flags", vp), ("stage_order", vp), ("epoch", u32), ("gated", i32),
                ("num_producers", i32), ("num_cus", i32), ("spin_limit", u32), ("error_word", vp),
                ("stage_counters", vp), ("split_ws", vp), ("split_ws_bytes", i64), ("epoch_ptr", vp)]


class GemmArArgs(C.Structure):
    _fields_ = [("A", vp), ("B", vp), ("C_final", vp), ("peer_src", vp), ("peer_recv", vp), ("M", i64), ("N", i64),
                ("K", i64), ("world", i32), ("flags", vp), ("stage_order", vp), ("epoch", u32), ("gated", i32),
                ("num_producers", i32), ("num_cus", i32), ("spin_limit", u32), ("error_word", vp),
                ("stage_counters", vp), ("done_flags", vp), ("split_ws", vp), ("split_ws_bytes", i64),
                ("epoch_ptr", vp)]


class GemmAr2Args(C.Structure):
    _fields_ = [("A", vp), ("B", vp), ("C_final", vp), ("sends", vp), ("peer_src", vp), ("peer_recv", vp),
                ("peer_reduced", vp), ("M", i64), ("N", i64), ("K", i64), ("world", i32), ("rank", i32),
                ("flags", vp), ("stage_order", vp), ("epoch", u32), ("gated", i32), ("num_producers", i32),
                ("num_cus", i32), ("spin_limit", u32), ("error_word", vp), ("stage_counters", vp),
                ("done_flags", vp), ("split_ws", vp), ("split_ws_bytes", i64), ("epoch_ptr", vp)]


class MoeIndex(C.Structure):
    _fields_ = [("padded_tokens_per_expert", vp), ("local_rb_per_expert", vp), ("pull_indices", vp),
                ("row_expert", vp), ("rb_expert", vp), ("rb_rows", vp), ("row_weight", vp), ("owner_offset", vp),
                ("row_to_slot", vp), ("row_to_owner", vp), ("slot_to_row", vp)]


class MoeIndexDevArgs(C.Structure):
    _fields_ = [("topk_ids", vp), ("topk_gates", vp), ("num_tokens", i32), ("topk", i32), ("expert_begin", i32),
                ("n_local", i32), ("row_block", i32), ("capacity_rows", i64), ("workspace", vp),
                ("workspace_bytes", i64), ("sizes", vp), ("out", MoeIndex)]


class MoePermuteArgs(C.Structure):
    _fields_ = [("tokens", vp), ("pull_indices", vp), ("post_tokens", vp), ("R_pad", i64), ("H", i64),
                ("n_src_rows", i64), ("tokens_per_src", i32), ("devs_per_node", i32), ("sizes", vp)]


class MoeGroupedGemmArgs(C.Structure):
    _fields_ = [("A", vp), ("W", vp), ("out", vp), ("rb_expert", vp), ("padded_tokens_per_expert", vp),
                ("rb_rows", vp), ("R_pad", i64), ("K", i64),
                ("Nw", i64), ("num_experts", i32), ("mode", i32), ("num_cus", i32), ("split_ws", vp),
                ("split_ws_bytes", i64), ("gather_pull", vp), ("n_src_rows", i64), ("tokens_per_src", i32),
                ("devs_per_node", i32), ("tile_n", i32), ("sizes", vp)]


class MoeCombineArgs(C.Structure):
    _fields_ = [("y_expert", vp), ("row_weight", vp), ("owner_offset", vp), ("slot_to_row", vp),
                ("y_out", vp), ("num_tokens", i64), ("H", i64), ("out_dtype", i32)]


class MoeFfnArgs(C.Structure):
    _fields_ = [("tokens", vp), ("pull_indices", vp), ("rb_expert", vp), ("padded_tokens_per_expert", vp),
                ("rb_rows", vp), ("row_weight", vp),
                ("owner_offset", vp), ("slot_to_row", vp), ("w1", vp), ("w2", vp), ("post_tokens", vp),
                ("act", vp), ("y_expert", vp), ("y_out", vp), ("num_tokens", i64), ("n_src_rows", i64),
                ("R_pad", i64), ("H", i64), ("I", i64), ("num_experts", i32), ("tokens_per_src", i32),
                ("devs_per_node", i32), ("out_dtype", i32), ("num_cus", i32), ("split_ws", vp),
                ("split_ws_bytes", i64), ("fuse_dispatch", i32), ("tile_n", i32),
                ("sizes", vp)]


_lib = None


def lib() -> C.CDLL:
    """Load libmk.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() "
                               "(or python -m mkernel_amd._build) first")
        L = C.CDLL(str(LIB_PATH))
        for name in ("mk_gemm", "mk_ag_gemm", "mk_ag_gemm_noalloc", "mk_gemm_rs", "mk_gemm_ar", "mk_gemm_ar_two_shot", "mk_moe_permute", "mk_moe_grouped_gemm",
                     "mk_moe_combine", "mk_moe_ffn_combine"):
            getattr(L, name).argtypes = [vp, vp]
            getattr(L, name).restype = C.c_int
        L.mk_moe_index_sizes.argtypes = [vp, i32, i32, i32, i32, i32, C.POINTER(i64), C.POINTER(i64)]
        L.mk_moe_index_sizes.restype = C.c_int
        L.mk_moe_build_indices.argtypes = [vp, vp, i32, i32, i32, i32, i32, C.POINTER(MoeIndex)]
        L.mk_moe_build_indices.restype = C.c_int
        L.mk_moe_index_workspace_bytes.argtypes = [i32, i32, i32]
        L.mk_moe_index_workspace_bytes.restype = i64
        L.mk_moe_build_indices_dev.argtypes = [vp, vp]
        L.mk_moe_build_indices_dev.restype = C.c_int
        L.mk_moe_invert_slots.argtypes = [vp, vp, i64, i32, i64, vp, vp, vp]
        L.mk_moe_invert_slots.restype = C.c_int
        L.mk_moe_tile_rows.argtypes = [vp, i64, vp, vp]
        L.mk_moe_tile_rows.restype = C.c_int
        L.mk_ag_gemm_noalloc_scratch_bytes.argtypes = []
        L.mk_ag_gemm_noalloc_scratch_bytes.restype = i64
        L.mk_query_workspace_bytes.argtypes = [i32, i64, i64, i64]
        L.mk_query_workspace_bytes.restype = i64
        L.mk_probe_mfma_ceiling.argtypes = [i64, i32, vp, vp, vp]
        L.mk_probe_mfma_ceiling.restype = C.c_int
        L.mk_probe_threads.argtypes = []
        L.mk_probe_threads.restype = i32
        L.mk_device_cu_count.argtypes = []
        L.mk_device_cu_count.restype = i32
        L.mk_last_error_string.argtypes = []
        L.mk_last_error_string.restype = C.c_char_p
        L.mk_epoch_advance.argtypes = [vp, vp]
        L.mk_epoch_advance.restype = i32
        L.mk_abi_version.argtypes = []
        L.mk_abi_version.restype = i32
        if L.mk_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI {L.mk_abi_version()}, this binding needs {ABI_VERSION}: "
                               "rebuild with __graft_entry__.build()")
        _lib = L
    return _lib


def check(fn: str, rc: int) -> None:
    if rc != 0:
        raise MkError(fn, rc, lib().mk_last_error_string().decode())


def call(fn: str, args: C.Structure, stream: int) -> None:
    check(fn, getattr(lib(), fn)(C.byref(args), vp(stream or None)))
