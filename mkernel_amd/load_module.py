"""The reference's operator modules, by name, on top of libmk.

``load(name)`` mirrors the reference loader (reference python/load_module.py:19-74):
it returns a module object exposing the same functions, argument names and
defaults as the reference's pybind modules, so a bench written against the
reference runs unchanged on one GPU:

=============================  ==============================================
name                           reference module definition
=============================  ==============================================
``ag_gemm``                    include/operators/ag_gemm/session.cuh:192-230
``gemm_rs``                    include/operators/gemm_rs/session.cuh:103-154
``gemm_ar``                    include/operators/gemm_ar/session.cuh:188-215
``dispatch_gemm``              include/operators/dispatch_gemm/session.cuh:89-133
``dispatch_gemm_glu_combine``  include/operators/dispatch_gemm_glu_combine/session.cuh:94-155
=============================  ==============================================

One GPU's share, no transport: the session functions (create_session,
get_fifo_handles, ...) are accepted and do nothing; FIFO / RDMA pointer
arguments are accepted and ignored.  What each operator reads and writes on
one GPU (which buffer holds the shards, the peer partials, the flags) is
spelled out on each function.  Every computation goes through libmk's C-ABI;
there is no fallback path.
"""
from __future__ import annotations

import types

import numpy as np
import torch

from . import ops

_DEFAULT_PRODUCERS = -1  # cooperative staging by the compute workgroups
_COUNTERS: dict = {}


def _counters(flags: torch.Tensor) -> torch.Tensor:
    """Piece counters for cooperative staging, one per flag word; zeroed once
    per flag buffer and kept for the life of the process."""
    key = (flags.data_ptr(), flags.numel())
    c = _COUNTERS.get(key)
    if c is None:
        c = torch.zeros(flags.numel(), dtype=torch.int32, device=flags.device)
        _COUNTERS[key] = c
    return c


class DistBuffer:
    """Reference ``DistBuffer`` (include/dist/parallel_buffer.cuh:87-120,
    391-414): ``.data_`` is the tensor, ``.local_rank_`` / ``.local_world_size_``
    the rank coordinates.  On one GPU it is a plain zero-initialised device
    allocation; ``local_rank`` names the rank whose share this GPU computes
    (it selects the owned slice in gemm_rs), not a device index."""

    def __init__(self, shape, dtype=torch.bfloat16, local_rank: int = 0, local_world_size: int = 1,
                 multicast: bool = False, backing: str = "vmm", device=None):
        if backing not in ("vmm", "cuda_malloc"):
            raise ValueError(f"unsupported backing {backing!r}")
        dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        self.data_ = torch.zeros(tuple(shape), dtype=dtype, device=dev)
        self.local_rank_ = int(local_rank)
        self.local_world_size_ = int(local_world_size)
        self.multicast_ = bool(multicast)


def _data(x):
    return x.data_ if isinstance(x, DistBuffer) else x


def _flags(barrier, n: int) -> torch.Tensor:
    f = _data(barrier).view(-1)
    if f.dtype != torch.int32:
        raise ValueError("barrier must be an int32 buffer")
    if f.numel() < n:
        raise ValueError(f"barrier holds {f.numel()} words, {n} flags needed")
    return f[:n]


class _Session:
    """Session helpers of the reference modules.  There is no proxy thread
    and no FIFO on one GPU: every call is accepted and returns the neutral
    value; set_epoch remembers the epoch."""

    def __init__(self):
        self.epoch = 1

    def create_session(self, *args, **kwargs):
        return None

    def destroy_session(self):
        return None

    def set_epoch(self, epoch: int):
        self.epoch = int(epoch)

    def prepare_epoch(self, *args, **kwargs):
        return None

    def commit_epoch(self, *args, **kwargs):
        return None

    def zero_recv_buf(self, *args, **kwargs):
        return None

    def get_fifo_handles(self):
        return (0, 0, 0, 0, 0)

    def get_arrival_flags_ptr(self):
        return 0

    def get_recv_buf_ptr(self):
        return 0

    def get_barrier_device_ptr(self):
        return 0

    def get_proxy_diagnostics(self):
        return []

    def get_proxy_timelines(self):
        return []


def _module(name: str, session: _Session, **fns) -> types.ModuleType:
    m = types.ModuleType(f"mkernel_amd_{name}")
    m.DistBuffer = DistBuffer
    for attr in ("create_session", "destroy_session", "set_epoch", "get_fifo_handles", "get_arrival_flags_ptr",
                 "get_recv_buf_ptr"):
        setattr(m, attr, getattr(session, attr))
    for k, v in fns.items():
        setattr(m, k, v)
    return m


# ---------------------------------------------------------------- ag_gemm ----
def _ag_module():
    s = _Session()

    def ag_gemm_multinode(A, B, C, barrier, recv_buf_ptr, fifo_triggers, fifo_head, fifo_tail, fifo_tail_cache,
                          fifo_capacity, arrival_flags_ptr, epoch, node_idx, num_comm_sms, a_half_bytes, A_recv,
                          active_sms=0, num_intra_comm_override=0, num_nodes=1, stage_order=None):
        """C = A_gathered @ B (reference include/operators/ag_gemm/ag_gemm.cuh:362-509).

        One GPU: ``A.data_`` [M, K] is the gathered A the GEMM reads;
        ``A_recv.data_`` [M, K] holds the row shards as they arrive (the
        producer role copies each 128-row tile into ``A.data_`` and publishes
        ``barrier`` word tile = epoch).  Pass ``A_recv=None`` when ``A.data_``
        is filled by someone else who also publishes the flags.  Producers:
        ``num_intra_comm_override`` dedicated producer workgroups if > 0,
        else cooperative staging: the compute workgroups copy the tiles
        between their tile rounds, the two XCD halves of the grid taking
        turns to copy ahead.  ``active_sms`` caps the grid (0 or >= CU
        count: every CU).  ``stage_order`` (int32 device tensor, optional)
        is the tile publication order the compute role follows."""
        Af = _data(A)
        M, K = Af.shape
        src = _data(A_recv) if A_recv is not None else None
        producers = (num_intra_comm_override if num_intra_comm_override > 0 else _DEFAULT_PRODUCERS) if src is not None else 0
        cus = ops.cu_count()
        grid = active_sms if 0 < active_sms < cus else 0
        fl = _flags(barrier, M // 128)
        ops.ag_gemm(src, Af, B, C, fl, stage_order, epoch=int(epoch), gated=True,
                    num_producers=producers, num_cus=grid, stage_counters=_counters(fl))
        return C

    return _module("ag_gemm", s, ag_gemm_multinode=ag_gemm_multinode,
                   get_proxy_diagnostics=s.get_proxy_diagnostics, get_proxy_timelines=s.get_proxy_timelines)


# ---------------------------------------------------------------- gemm_rs ----
def _rs_module():
    s = _Session()

    def gemm_rs_fused(A, B, workspace, output, barrier, ready, recv_buf_ptr, staging_buf_ptr, fifo_triggers,
                      fifo_head, fifo_tail, fifo_tail_cache, fifo_capacity, arrival_flags_ptr, epoch, node_idx,
                      num_comp_sms, num_intra_comm, num_send_sms, num_reduce_sms, use_acquire_poll,
                      reduce_poll_sleep_ns, ready_chunk, staging, num_nodes=1, stage_order=None):
        """Row-parallel GEMM + reduce-scatter (reference
        include/operators/gemm_rs/gemm_rs.cuh:510-935).

        One GPU, rank r = ``output.local_rank_``, world = M / output rows:
        ``workspace.data_`` [M, N] receives this rank's partial for every
        row it does not own (the would-be sends); ``output.data_`` [M/world,
        N] = own partial + sum of the world-1 peer partials (fp32 adds, one
        bf16 rounding).  Peer partials arrive in ``staging.data_`` [world-1,
        M/world, N]; the producer role copies them to the device buffer at
        ``recv_buf_ptr`` (same shape) and publishes ``barrier`` words; the
        epilogue of each owned tile waits for its peers' words.
        ``staging=None`` means the partials are already at ``recv_buf_ptr``
        and ``barrier`` is published by someone else."""
        out = _data(output)
        M, N = A.shape[0], B.shape[1]
        rows = out.shape[0]
        world = M // rows
        rank = output.local_rank_ if isinstance(output, DistBuffer) else 0
        if world * rows != M:
            raise ValueError("output rows must divide M")
        nflags = (world - 1) * rows // 128
        recv = None
        if world > 1:
            if not recv_buf_ptr:
                raise ValueError("recv_buf_ptr must point at the [world-1, M/world, N] receive buffer")
            recv = _DevicePtr(int(recv_buf_ptr))
        src = _data(staging) if staging is not None else None
        producers = (num_intra_comm if num_intra_comm > 0 else _DEFAULT_PRODUCERS) if src is not None else 0
        fl = _flags(barrier, max(nflags, 1))
        ops.gemm_rs(A, B, _data(workspace), out, src, recv, world, rank, fl, stage_order, epoch=int(epoch),
                    gated=True, num_producers=producers, stage_counters=_counters(fl))
        return out

    return _module("gemm_rs", s, gemm_rs_fused=gemm_rs_fused, prepare_epoch=s.prepare_epoch,
                   commit_epoch=s.commit_epoch, zero_recv_buf=s.zero_recv_buf)


# ---------------------------------------------------------------- gemm_ar ----
def _ar_module():
    s = _Session()

    def gemm_ar_multinode(A, B, C, barrier, C_final, staging_buf_ptr, recv_buf_ptr, fifo_triggers, fifo_head,
                          fifo_tail, fifo_tail_cache, fifo_capacity, arrival_flags_ptr, epoch, node_idx,
                          num_intra_comm_sms, num_inter_comm_sms, ar_done_ptr, num_nodes=1, stage_order=None,
                          **kwargs):
        """GEMM + all-reduce (reference include/operators/gemm_ar/session.cuh:188-215,
        src/gemm_ar.cu).

        One GPU, world = ``C.local_world_size_``: ``C_final.data_`` [M, N] =
        A @ B + the sum of the world-1 peer partials (fp32 adds, one bf16
        rounding).  The partials to stage are at ``staging_buf_ptr``
        [world-1, M, N] (device address; 0 = already in place); the
        producer role copies them to ``recv_buf_ptr`` (same shape) and
        publishes ``barrier`` words; each output tile is published in
        ``ar_done_ptr`` (int32 [(M/256) * (N/256)], 0 = none) with the
        epoch.  ``C`` is the rank's partial in the reference's multicast
        buffer; on one GPU it is not written.  Remaining reference keyword
        arguments (queues, tracing, RDMA) are accepted and ignored."""
        Cf = _data(C_final)
        M, N = A.shape[0], B.shape[1]
        world = C.local_world_size_ if isinstance(C, DistBuffer) else 1
        nflags = (world - 1) * M // 128
        recv = _DevicePtr(int(recv_buf_ptr)) if world > 1 and recv_buf_ptr else None
        if world > 1 and recv is None:
            raise ValueError("recv_buf_ptr must point at the [world-1, M, N] receive buffer")
        src = _DevicePtr(int(staging_buf_ptr)) if staging_buf_ptr else None
        producers = (num_intra_comm_sms if num_intra_comm_sms > 0 else _DEFAULT_PRODUCERS) if src is not None else 0
        fl = _flags(barrier, max(nflags, 1))
        done = _DevicePtr(int(ar_done_ptr)) if ar_done_ptr else None
        ops.gemm_ar(A, B, Cf, src, recv, world, fl, stage_order, epoch=int(epoch), gated=world > 1,
                    num_producers=producers, stage_counters=_counters(fl), done_flags=done)
        return Cf

    return _module("gemm_ar", s, gemm_ar_multinode=gemm_ar_multinode, get_barrier_device_ptr=s.get_barrier_device_ptr)


class _DevicePtr:
    """A raw device address passed where the C-ABI wants a pointer."""

    def __init__(self, ptr: int):
        self.ptr = ptr

    def data_ptr(self) -> int:
        return self.ptr


# ---------------------------------------------------------- dispatch_gemm ----
def _dispatch_module():
    s = _Session()

    def moe_dispatch_gemm_fused(pre_tokens, peer_tokens, copy_ready, post_tokens, weights, outputs,
                                padded_tokens_per_expert, pull_dispatch_indices, local_rb_per_expert, barrier,
                                sync_barrier, recv_buf_ptr, fifo_triggers, fifo_head, fifo_tail, fifo_tail_cache,
                                fifo_capacity, arrival_flags_ptr, epoch, node_idx, num_local_tokens,
                                num_padded_local_tokens, num_send_sms, num_copy_sms, num_comm_sms_intra,
                                num_nodes=1):
        """Token permute + grouped GEMM (reference
        include/operators/dispatch_gemm/dispatch_gemm.cuh:238-387).

        ``post_tokens[r] = pre_tokens.data_[pull_dispatch_indices[r, 2]]``
        (zero rows for padding), then ``outputs[rows_e] = post_tokens[rows_e]
        @ weights[e]`` per local expert, expert ranges taken from
        ``padded_tokens_per_expert``."""
        tok = _data(pre_tokens)[:num_local_tokens]
        post = post_tokens[:num_padded_local_tokens]
        rb_rows = torch.empty(max(num_padded_local_tokens // 128, 1), dtype=torch.int32, device=post.device)
        ops.moe_tile_rows(pull_dispatch_indices[:num_padded_local_tokens], rb_rows)
        ops.moe_permute(tok, pull_dispatch_indices, post, tokens_per_src=num_local_tokens)
        ops.moe_grouped_gemm(post, weights, outputs[:num_padded_local_tokens],
                             padded_tokens_per_expert=padded_tokens_per_expert, mode=0, rb_rows=rb_rows)
        return outputs

    return _module("dispatch_gemm", s, moe_dispatch_gemm_fused=moe_dispatch_gemm_fused)


# ------------------------------------------------ dispatch_gemm_glu_combine ----
def _glu_module():
    s = _Session()

    def moe_dispatch_gemm_glu_combine_fused(pre_tokens, peer_tokens, copy_ready, post_tokens, w1, w2, act, y_expert,
                                            row_expert, topk_weights, padded_tokens_per_expert, pull_dispatch_indices,
                                            local_rb_per_expert, barrier, sync_barrier, y_out, comb_buf, owner_offset,
                                            row_to_slot, row_to_owner, inter_comb_buf, inter_owner_offset,
                                            inter_row_to_slot, inter_row_to_owner, use_inter_gather, recv_buf_ptr,
                                            fifo_triggers, fifo_head, fifo_tail, fifo_tail_cache, fifo_capacity,
                                            arrival_flags_ptr, epoch, node_idx, num_local_tokens,
                                            num_padded_local_tokens, num_send_sms, num_copy_sms, num_comm_sms_intra,
                                            use_gather, num_nodes=1, cross_node_barrier_ptr=0):
        """Permute -> GEMM1 + SwiGLU -> GEMM2 -> top-k weighted combine
        (reference include/operators/dispatch_gemm_glu_combine/dispatch_gemm_glu_combine.cuh:307-548).

        Writes post_tokens, act, y_expert and ``y_out.data_`` [num_local_tokens,
        H] (fp32 or bf16) = sum over each token's rows of topk_weights[r] *
        y_expert[r], gathered through owner_offset / row_to_slot (the CSR the
        reference's build_gather_indices produces).  y_out is overwritten, so
        the reference's zeroing before each call is harmless but not needed."""
        tok = _data(pre_tokens)[:num_local_tokens]
        yo = _data(y_out)
        R_pad = num_padded_local_tokens
        # every slot index is < R <= R_pad, so R_pad entries always suffice
        slot_to_row = torch.empty(max(R_pad, 1), dtype=torch.int32, device=row_to_slot.device)
        ops.moe_invert_slots(row_to_slot[:R_pad], row_to_owner[:R_pad], slot_to_row)
        rb_rows = torch.empty(max(R_pad // 128, 1), dtype=torch.int32, device=row_to_slot.device)
        ops.moe_tile_rows(pull_dispatch_indices[:R_pad], rb_rows)
        ops.moe_ffn_combine(tok, pull_dispatch_indices, topk_weights, owner_offset, slot_to_row, w1, w2,
                            post_tokens[:R_pad], act[:R_pad], y_expert[:R_pad], yo[:num_local_tokens],
                            padded_tokens_per_expert=padded_tokens_per_expert, tokens_per_src=num_local_tokens,
                            rb_rows=rb_rows)
        return yo

    return _module("dispatch_gemm_glu_combine", s, moe_dispatch_gemm_glu_combine_fused=moe_dispatch_gemm_glu_combine_fused,
                   get_barrier_device_ptr=s.get_barrier_device_ptr)


_BUILDERS = {
    "ag_gemm": _ag_module,
    "gemm_rs": _rs_module,
    "gemm_ar": _ar_module,
    "dispatch_gemm": _dispatch_module,
    "dispatch_gemm_glu_combine": _glu_module,
}


def load(name: str) -> types.ModuleType:
    """Return the operator module ``name`` (reference python/load_module.py:19)."""
    if name not in _BUILDERS:
        raise RuntimeError(f"unknown operator module {name!r}; available: {sorted(_BUILDERS)}")
    return _BUILDERS[name]()


def build_routing_indices(topk_ids: np.ndarray, gates: np.ndarray, rank: int, experts: int, ep: int,
                          row_block: int = 128) -> dict:
    """The host-side index tables the reference benches build in Python
    (bench/dispatch_gemm_bench.py:127-188, bench/dispatch_gemm_glu_combine_bench.py:222-293)
    for the rank that owns experts [rank*experts/ep, (rank+1)*experts/ep),
    computed by libmk's C++ builder."""
    n_local = experts // ep
    return ops.moe_build_indices(topk_ids, gates, rank * n_local, n_local, row_block)
