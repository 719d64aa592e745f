"""The reference's operator modules, by name, on top of libmk.

``load(name)`` mirrors the reference loader (reference python/load_module.py:19-74):
it returns a module object exposing the same functions, argument names and
defaults as the reference's pybind modules:

=============================  ==============================================
name                           reference module definition
=============================  ==============================================
``ag_gemm``                    include/operators/ag_gemm/session.cuh:192-230
``gemm_rs``                    include/operators/gemm_rs/session.cuh:103-154
``gemm_ar``                    include/operators/gemm_ar/session.cuh:140-215
``dispatch_gemm``              include/operators/dispatch_gemm/session.cuh:89-133
``dispatch_gemm_glu_combine``  include/operators/dispatch_gemm_glu_combine/session.cuh:94-155
=============================  ==============================================

The buffers take the roles the reference benches give them
(bench/ag_gemm_bench.py:364-384, bench/gemm_rs_bench.py:742-766,
bench/gemm_ar_bench.py:429-470): the caller's own data sits where the
reference bench writes it, and buffers the bench zeroes before every call
(``A_recv``, ``barrier``, ``staging``, ``C`` of gemm_ar) are never read.
The rank's place in the node is the ``local_rank_`` / ``local_world_size_``
of its DistBuffers.  With ``local_world_size_ == 1`` (one process, the only
world one GPU can run) a reference bench runs unchanged and every result is
the reference's.  A rank of a larger world can be emulated on one GPU: what
the peers would deliver over xGMI is passed as one extra keyword
(``peer_shards`` for ag_gemm, ``peer_partials`` for gemm_rs / gemm_ar) and
the in-GPU producer role stages it; without it such a call raises, since
the data it needs does not exist on this GPU.

Each module has one session.  The session owns the producer role's flag
array (``get_arrival_flags_ptr``), its piece counters, the receive buffer
for staged peer partials (``get_recv_buf_ptr``) and the launch epoch: every
call stamps its flags with a fresh epoch, so flags are never reset and a
caller that keeps ``epoch`` fixed (bench/ag_gemm_bench.py:355-357) is still
gated correctly.  Calls of one module on different streams at once would
share those flags and race, as the reference's module statics do
(include/operators/ag_gemm/session.cuh:13-20).  FIFO / RDMA arguments are
accepted and ignored; multi-node calls (``num_nodes > 1``) raise.  Every
computation goes through libmk's C-ABI; there is no fallback path.
"""
from __future__ import annotations

import types

import numpy as np
import torch

from . import ops

# Producer-role flags (and piece counters) per device: one word per staged
# 128-row block.  Config-sized calls need at most a few thousand.
_FLAG_WORDS = 1 << 16


def _cu_clamp(active_sms) -> int:
    """Persistent grid for a reference ``active_sms``: 0 or at least the CU
    count means every CU (the reference passes the device's SM count,
    bench/ag_gemm_bench.py:375-376)."""
    cus = ops.cu_count()
    a = int(active_sms or 0)
    return a if 0 < a < cus else 0


class DistBuffer:
    """Reference ``DistBuffer`` (include/dist/parallel_buffer.cuh:391-414),
    both constructors: ``DistBuffer(tensor, local_rank, local_world_size,
    multicast=False)`` wraps a tensor, ``DistBuffer(shape, dtype, local_rank,
    local_world_size, multicast=False, backing="vmm")`` allocates a zeroed
    device buffer.  ``.data_`` / ``.data()`` is the tensor, ``.local_rank_`` /
    ``.local_world_size_`` the rank's place in the node.  On one GPU it is a
    plain device allocation (no peer mapping, no multicast)."""

    def __init__(self, shape_or_tensor, *args, **kwargs):
        if isinstance(shape_or_tensor, torch.Tensor):
            names = ("local_rank", "local_world_size", "multicast")
            vals = dict(zip(names, args), **kwargs)
            if set(vals) - set(names):
                raise TypeError(f"unexpected arguments {sorted(set(vals) - set(names))}")
            self.data_ = shape_or_tensor
        else:
            names = ("dtype", "local_rank", "local_world_size", "multicast", "backing", "device")
            vals = dict(zip(names, args), **kwargs)
            if set(vals) - set(names):
                raise TypeError(f"unexpected arguments {sorted(set(vals) - set(names))}")
            backing = vals.get("backing", "vmm")
            if backing not in ("vmm", "cuda_malloc"):
                raise ValueError(f"unsupported backing {backing!r}")
            dev = vals.get("device")
            dev = torch.device("cuda", torch.cuda.current_device()) if dev is None else torch.device(dev)
            self.data_ = torch.zeros(tuple(shape_or_tensor), dtype=vals.get("dtype", torch.bfloat16), device=dev)
        self.local_rank_ = int(vals.get("local_rank", 0))
        self.local_world_size_ = int(vals.get("local_world_size", 1))
        self.multicast_ = bool(vals.get("multicast", False))
        if not 0 <= self.local_rank_ < max(self.local_world_size_, 1):
            raise ValueError(f"local_rank {self.local_rank_} outside local_world_size {self.local_world_size_}")

    def data(self):
        return self.data_

    @property
    def multicast_enabled(self) -> bool:
        return False

    @property
    def multicast_ptr_u64(self) -> int:
        return 0


def _data(x):
    return x.data_ if isinstance(x, DistBuffer) else x


def _place(*bufs) -> tuple:
    """(local_rank, local_world_size) of the first DistBuffer among bufs;
    (0, 1) when none is one."""
    for b in bufs:
        if isinstance(b, DistBuffer):
            return b.local_rank_, max(b.local_world_size_, 1)
    return 0, 1


def _single_node(num_nodes) -> None:
    if int(num_nodes) != 1:
        raise ValueError(f"num_nodes={num_nodes}: multi-node transport is not part of this library (one GPU)")


class _Session:
    """Session of one operator module.  The reference's session helpers
    (create_session, get_fifo_handles, ...) do nothing here but keep their
    names and return shapes; the session owns the producer role's flag
    array, piece counters, receive buffer and launch epoch per device."""

    def __init__(self):
        self.epoch = 1          # the caller's epoch (set_epoch / argument), recorded only
        self._dev = {}          # device index -> dict of library-owned buffers
        self._checked = set()   # table versions already validated

    # ---- library-owned device state ----
    def _state(self, dev: torch.device) -> dict:
        i = dev.index if dev.index is not None else torch.cuda.current_device()
        st = self._dev.get(i)
        if st is None:
            d = torch.device("cuda", i)
            st = {"flags": torch.zeros(_FLAG_WORDS, dtype=torch.int32, device=d),
                  "counters": torch.zeros(_FLAG_WORDS, dtype=torch.int32, device=d),
                  "launch": 0, "recv": None, "order": {}, "tables": {}}
            self._dev[i] = st
        return st

    def flags(self, n: int, dev) -> tuple:
        """(flags[:n], counters[:n]) on dev: zeroed once, never reset."""
        if n > _FLAG_WORDS:
            raise ValueError(f"{n} flag words needed, the session holds {_FLAG_WORDS}")
        st = self._state(dev)
        return st["flags"][:n], st["counters"][:n]

    def next_epoch(self, dev) -> int:
        """A fresh flag epoch for one launch on dev (1, 2, ...; never 0)."""
        st = self._state(dev)
        st["launch"] = st["launch"] % 0x7FFFFFFF + 1
        return st["launch"]

    def recv(self, shape, dev) -> torch.Tensor:
        """The receive buffer for staged peer partials (bf16, grown on demand)."""
        st = self._state(dev)
        n = int(np.prod(shape))
        if st["recv"] is None or st["recv"].numel() < n:
            st["recv"] = torch.zeros(n, dtype=torch.bfloat16, device=dev)
        return st["recv"][:n].view(tuple(shape))

    def buffer(self, key, n: int, dev) -> torch.Tensor:
        """A cached int32 device buffer of at least n entries (no allocation
        once it exists)."""
        st = self._state(dev)
        b = st["tables"].get(key)
        if b is None or b.numel() < n:
            b = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
            st["tables"][key] = b
        return b[:n]

    def checked(self, key) -> bool:
        """True if `key` was validated before; records it (a failed check
        raises before the next call asks again, so it is re-checked)."""
        if key in self._checked:
            return True
        self._checked.add(key)
        return False

    def unchecked(self, key) -> None:
        self._checked.discard(key)

    def stage_order(self, n: int, present: range, order, dev) -> torch.Tensor:
        """Device stage order: the blocks in `present` first (ascending), then
        the others in the order of `order` (a permutation of range(n), host or
        device; None = ascending).  Cached per (n, present, order tensor)."""
        key = (n, present.start, present.stop, None if order is None else
               (order.data_ptr(), order._version, order.numel(), str(order.device)))
        st = self._state(dev)
        t = st["order"].get(key)
        if t is None:
            perm = np.arange(n) if order is None else np.asarray(order.cpu() if torch.is_tensor(order) else order)
            if sorted(perm.tolist()) != list(range(n)):
                raise ValueError("stage_order must be a permutation of the 128-row blocks")
            rest = [int(b) for b in perm if int(b) not in present]
            t = torch.tensor(list(present) + rest, dtype=torch.int32, device=dev)
            st["order"][key] = t
        return t

    # ---- reference session helpers ----
    def create_session(self, *args, **kwargs):
        return None

    def destroy_session(self):
        return None

    def set_epoch(self, epoch: int):
        self.epoch = int(epoch)

    def prepare_epoch(self, *args, **kwargs):
        return None

    def commit_epoch(self, epoch=None, *args, **kwargs):
        if epoch is not None:
            self.epoch = int(epoch)

    def zero_recv_buf(self, *args, **kwargs):
        return None

    def reset_arrival_flags(self, *args, **kwargs):
        """Flags carry a fresh epoch per launch and are never reset."""
        return None

    def get_fifo_handles(self):
        return (0, 0, 0, 0, 0)

    def get_arrival_flags_ptr(self):
        """Device address of the producer role's flag array on the current
        device (int32 words, flag = launch epoch once the block is staged);
        0 without a GPU."""
        if not torch.cuda.is_available():
            return 0
        return self._state(torch.device("cuda", torch.cuda.current_device()))["flags"].data_ptr()

    def get_recv_buf_ptr(self):
        """Device address of the staged-peer-partials buffer (0 until a call
        that stages partials has allocated it)."""
        if not torch.cuda.is_available():
            return 0
        st = self._dev.get(torch.cuda.current_device())
        return 0 if st is None or st["recv"] is None else st["recv"].data_ptr()

    def get_barrier_device_ptr(self):
        return 0

    def get_arrival_tails_ptr(self):
        return 0

    def get_num_qps(self):
        return 0

    def get_ready_queue_handles(self):
        return (0, 0, 0, 0)

    def set_ready_queue_total(self, total):
        return None

    def get_globaltimer_calibration(self, *args, **kwargs):
        return (0, 0)

    def get_proxy_diagnostics(self):
        return []

    def get_proxy_timelines(self):
        return []


def _module(name: str, session: _Session, helpers, **fns) -> types.ModuleType:
    m = types.ModuleType(f"mkernel_amd_{name}")
    m.DistBuffer = DistBuffer
    for attr in ("create_session", "destroy_session", "set_epoch", "get_fifo_handles", "get_arrival_flags_ptr",
                 "get_recv_buf_ptr", *helpers):
        setattr(m, attr, getattr(session, attr))
    for k, v in fns.items():
        setattr(m, k, v)
    return m


def _producers(dedicated: int) -> int:
    """libmk producer mode for a reference intra-comm SM count: cooperative
    staging by the compute workgroups (-1, the fastest mode at every config
    measured) unless dedicated producer workgroups are asked for."""
    return int(dedicated) if dedicated and dedicated > 0 else -1


# ---------------------------------------------------------------- ag_gemm ----
def _ag_module():
    s = _Session()

    def ag_gemm_multinode(A, B, C, barrier, recv_buf_ptr, fifo_triggers, fifo_head, fifo_tail, fifo_tail_cache,
                          fifo_capacity, arrival_flags_ptr, epoch, node_idx, num_comm_sms, a_half_bytes, A_recv,
                          active_sms=132, num_intra_comm_override=0, num_nodes=1, *, peer_shards=None,
                          stage_order=None, dedicated_producers=0):
        """C = A_gathered @ B (reference include/operators/ag_gemm/ag_gemm.cuh:362-509).

        ``A.data_`` [M, K] is the node's gathered A; this rank's shard (rows
        [r*M/W, (r+1)*M/W), r / W = ``A.local_rank_`` / ``local_world_size_``)
        is already there, written by the caller as the reference bench does
        (bench/ag_gemm_bench.py:364-372).  The other shards arrive while the
        GEMM runs: ``peer_shards`` ([M, K], tensor or DistBuffer; only rows
        outside this rank's shard are read) stands in for the peers, and the
        producer role copies each of their 128-row blocks into ``A.data_``
        and publishes its flag; the compute role gates every tile on its
        rows' flags.  The own shard's flags are published without a copy.
        ``stage_order``: the order the peer blocks arrive in (a permutation
        of the M/128 blocks; own blocks are dropped from it).  ``A_recv`` is
        the reference's inter-node receive buffer (empty on one node) and
        ``barrier`` its intra-node flag buffer: neither is read or written;
        the flags are the session's (``get_arrival_flags_ptr``).
        ``num_intra_comm_override`` / ``num_comm_sms`` (the reference's SM
        split) select nothing: the blocks are staged cooperatively by the
        compute workgroups, unless ``dedicated_producers`` > 0 asks for that
        many producer workgroups.  ``active_sms`` caps the persistent grid
        at that many workgroups (0 or >= the CU count: every CU).  Its
        default is the reference's, 132 (include/operators/ag_gemm/
        session.cuh:227), so a call that relies on it runs on 132 of the
        MI355X's 256 CUs, as it runs on 132 SMs on any reference GPU; the
        reference benches pass the device's full count
        (bench/ag_gemm_bench.py:375-376)."""
        _single_node(num_nodes)
        s.epoch = int(epoch)
        Af = _data(A)
        M, K = Af.shape
        rank, world = _place(A)
        if M % (128 * world):
            raise ValueError(f"M={M} must be a multiple of 128 * local_world_size ({world})")
        grid = _cu_clamp(active_sms)
        if world == 1:
            # every row is this rank's: nothing arrives, nothing to gate on
            ops.ag_gemm(None, Af, B, C, None, None, epoch=1, gated=False, num_producers=0, num_cus=grid)
            return C
        if peer_shards is None:
            raise ValueError("ag_gemm_multinode on one GPU with local_world_size > 1: pass the shards the peers "
                             "would deliver as peer_shards=[M, K] (only rows outside this rank's shard are read)")
        src = _data(peer_shards)
        if tuple(src.shape) != (M, K) or src.dtype != Af.dtype:
            raise ValueError(f"peer_shards must be {tuple(Af.shape)} {Af.dtype}")
        nb = M // 128
        per = nb // world
        present = range(rank * per, (rank + 1) * per)
        order = s.stage_order(nb, present, stage_order, Af.device)
        fl, cnt = s.flags(nb, Af.device)
        ops.ag_gemm(src, Af, B, C, fl, order, epoch=s.next_epoch(Af.device), gated=True,
                    num_producers=_producers(dedicated_producers), num_cus=grid, stage_counters=cnt,
                    n_present=per)
        return C

    return _module("ag_gemm", s, ("get_proxy_diagnostics", "get_proxy_timelines"),
                   ag_gemm_multinode=ag_gemm_multinode)


# ---------------------------------------------------------------- gemm_rs ----
def _rs_module():
    s = _Session()

    def gemm_rs_fused(A, B, workspace, output, barrier, ready, recv_buf_ptr, staging_buf_ptr, fifo_triggers,
                      fifo_head, fifo_tail, fifo_tail_cache, fifo_capacity, arrival_flags_ptr, epoch, node_idx,
                      num_comp_sms, num_intra_comm, num_send_sms, num_reduce_sms, use_acquire_poll,
                      reduce_poll_sleep_ns, ready_chunk, staging, num_nodes=1, *, peer_partials=None,
                      stage_order=None, dedicated_producers=0):
        """Row-parallel GEMM + reduce-scatter (reference
        include/operators/gemm_rs/gemm_rs.cuh:510-935).

        Rank r of W (``output.local_rank_`` / ``local_world_size_``) owns
        rows [r*M/W, (r+1)*M/W): ``output.data_`` [M/W, N] = its own partial
        A[owned] @ B + the W-1 peers' partials for those rows (fp32 adds in
        rank order, one bf16 rounding); ``workspace.data_`` [M, N] receives
        this rank's partial of every row it does not own (the would-be
        sends).  The peers' partials, [W-1, M/W, N] in rank order without r,
        are passed as ``peer_partials``; the producer role stages them into
        the session's receive buffer (``get_recv_buf_ptr``) and publishes a
        flag per 128-row block, and each owned tile's epilogue waits for its
        blocks.  ``staging`` (the reference's store_add accumulation buffer,
        src/gemm_rs.cu:74-93), ``staging_buf_ptr``, ``recv_buf_ptr``,
        ``barrier``, ``ready`` and ``ready_chunk`` are not read or written.
        The SM-split arguments select nothing (cooperative staging by the
        compute workgroups, or ``dedicated_producers`` producer workgroups).
        With W == 1 the output is A @ B."""
        _single_node(num_nodes)
        s.epoch = int(epoch)
        out = _data(output)
        M, N = A.shape[0], B.shape[1]
        rank, world = _place(output, workspace)
        rows = out.shape[0]
        if rows * world != M:
            raise ValueError(f"output has {rows} rows; M={M} over local_world_size {world} needs {M // world}")
        ws = _data(workspace)
        if world == 1:
            ops.gemm_rs(A, B, ws, out, None, None, 1, 0, None, None, epoch=1, gated=False, num_producers=0)
            return out
        if peer_partials is None:
            raise ValueError("gemm_rs_fused on one GPU with local_world_size > 1: pass the partials the peers "
                             f"would send as peer_partials=[{world - 1}, {rows}, {N}] (rank order, own rank left out)")
        src = _data(peer_partials)
        if tuple(src.shape) != (world - 1, rows, N) or src.dtype != torch.bfloat16:
            raise ValueError(f"peer_partials must be ({world - 1}, {rows}, {N}) bf16")
        dev = out.device
        nflags = (world - 1) * rows // 128
        recv = s.recv((world - 1, rows, N), dev)
        fl, cnt = s.flags(nflags, dev)
        order = None if stage_order is None else s.stage_order(nflags, range(0), stage_order, dev)
        ops.gemm_rs(A, B, ws, out, src, recv, world, rank, fl, order, epoch=s.next_epoch(dev), gated=True,
                    num_producers=_producers(dedicated_producers), stage_counters=cnt)
        return out

    return _module("gemm_rs", s, ("prepare_epoch", "commit_epoch", "zero_recv_buf"), gemm_rs_fused=gemm_rs_fused)


# ---------------------------------------------------------------- gemm_ar ----
class _DevicePtr:
    """A raw device address passed where the C-ABI wants a pointer."""

    def __init__(self, ptr: int):
        self.ptr = ptr

    def data_ptr(self) -> int:
        return self.ptr


def _ar_module():
    s = _Session()

    def gemm_ar_multinode(A, B, C, barrier, C_final, staging_buf_ptr, recv_buf_ptr, fifo_triggers, fifo_head,
                          fifo_tail, fifo_tail_cache, fifo_capacity, arrival_flags_ptr, epoch, node_idx,
                          num_intra_comm_sms, num_inter_comm_sms, ar_done_ptr, num_nodes=1, *, peer_partials=None,
                          stage_order=None, dedicated_producers=0, **kwargs):
        """GEMM + all-reduce (reference include/operators/gemm_ar/session.cuh:188-215,
        src/gemm_ar.cu).

        Rank r of W (``C.local_world_size_``): ``C_final.data_`` [M, N] =
        A @ B + the W-1 peers' partials (fp32 adds in rank order, one bf16
        rounding), the reference's all_reduce(matmul)
        (bench/gemm_ar_bench.py:510-514).  The peers' partials, [W-1, M, N]
        in rank order without r, are passed as ``peer_partials``; the
        producer role stages them into the session's receive buffer and
        publishes a flag per 128-row block, and each output tile waits for
        its blocks.  When ``ar_done_ptr`` is non-zero, word t = row_tile *
        (N/256) + col_tile of it (int32) is set to the launch's epoch (non-zero)
        once that 256x256 tile of C_final is final.  ``C`` (the reference's
        multicast partial buffer), ``staging_buf_ptr``, ``recv_buf_ptr`` and
        ``barrier`` are not read or written; the remaining reference keyword
        arguments (queues, RDMA, tracing) are accepted and ignored."""
        _single_node(num_nodes)
        s.epoch = int(epoch)
        Cf = _data(C_final)
        M, N = A.shape[0], B.shape[1]
        rank, world = _place(C, C_final)
        dev = Cf.device
        done = _DevicePtr(int(ar_done_ptr)) if ar_done_ptr else None
        if world == 1:
            ops.gemm_ar(A, B, Cf, None, None, 1, None, None, epoch=s.next_epoch(dev), gated=False, done_flags=done)
            return Cf
        if peer_partials is None:
            raise ValueError("gemm_ar_multinode on one GPU with local_world_size > 1: pass the partials the peers "
                             f"would send as peer_partials=[{world - 1}, {M}, {N}] (rank order, own rank left out)")
        src = _data(peer_partials)
        if tuple(src.shape) != (world - 1, M, N) or src.dtype != torch.bfloat16:
            raise ValueError(f"peer_partials must be ({world - 1}, {M}, {N}) bf16")
        nflags = (world - 1) * M // 128
        recv = s.recv((world - 1, M, N), dev)
        fl, cnt = s.flags(nflags, dev)
        order = None if stage_order is None else s.stage_order(nflags, range(0), stage_order, dev)
        ops.gemm_ar(A, B, Cf, src, recv, world, fl, order, epoch=s.next_epoch(dev), gated=True,
                    num_producers=_producers(dedicated_producers), stage_counters=cnt, done_flags=done)
        return Cf

    return _module("gemm_ar", s, ("get_barrier_device_ptr", "reset_arrival_flags", "get_arrival_tails_ptr",
                                  "get_num_qps", "get_ready_queue_handles", "set_ready_queue_total",
                                  "get_globaltimer_calibration", "get_proxy_diagnostics", "get_proxy_timelines"),
                   gemm_ar_multinode=gemm_ar_multinode)


# ---------------------------------------------------------------- MoE ----
def _local_tables(s: _Session, pre_tokens, pull, padded, n_experts: int, R_pad: int, node_idx: int,
                  num_nodes, validate: bool = True) -> torch.Tensor:
    """Checks that the routing tables describe one GPU's layout (every pulled
    token is on this GPU) and returns the per-local-expert padded row counts.
    The reference's padded table lists every expert of the job
    (bench/dispatch_gemm_bench.py:161-166,280); the local slice starts at
    this GPU's first expert.  Table contents are checked once per tensor
    version (one host read-back, which synchronizes the stream);
    ``validate=False`` skips that check."""
    _single_node(num_nodes)
    rank, world = _place(pre_tokens)
    if world != 1 or int(node_idx) != 0:
        raise ValueError("MoE dispatch on one GPU takes one-process tables (local_world_size 1, node 0); "
                         "rows pulled from other GPUs need the xGMI/RDMA transport, which is not part of this library")
    dev = pull.device
    if padded.numel() == n_experts:
        pl = padded
    elif padded.numel() % n_experts == 0 and padded.numel() // n_experts > rank:
        pl = padded[rank * n_experts:(rank + 1) * n_experts]
    else:
        raise ValueError(f"padded_tokens_per_expert has {padded.numel()} entries for {n_experts} local experts")
    key = ("tables", str(dev), pull.data_ptr(), pull._version, padded.data_ptr(), padded._version, R_pad)
    if validate and not s.checked(key):
        p = pull[:R_pad].cpu().numpy()
        real = p[:, 0] >= 0
        bad = None
        if (p[real, 0] != 0).any() or (p[real, 1] != 0).any():
            bad = "pull_dispatch_indices names tokens of other GPUs (src_node/src_dev != 0)"
        elif int(pl.sum()) != R_pad:
            bad = f"the local experts' padded rows sum to {int(pl.sum())}, not num_padded_local_tokens={R_pad}"
        if bad:
            s.unchecked(key)
            raise ValueError(bad)
    return pl


def _dispatch_module():
    s = _Session()

    def moe_dispatch_gemm_fused(pre_tokens, peer_tokens, copy_ready, post_tokens, weights, outputs,
                                padded_tokens_per_expert, pull_dispatch_indices, local_rb_per_expert, barrier,
                                sync_barrier, recv_buf_ptr, fifo_triggers, fifo_head, fifo_tail, fifo_tail_cache,
                                fifo_capacity, arrival_flags_ptr, epoch, node_idx, num_local_tokens,
                                num_padded_local_tokens, num_send_sms, num_copy_sms, num_comm_sms_intra,
                                num_nodes=1, *, write_post_tokens=False, validate_tables=True):
        """Token dispatch + grouped GEMM (reference
        include/operators/dispatch_gemm/dispatch_gemm.cuh:238-387).

        ``outputs[r] = pre_tokens.data_[pull_dispatch_indices[r, 2]] @
        weights[e(r)]`` for the first ``num_padded_local_tokens`` rows (zero
        rows for padding), e(r) from the local experts' padded row counts.
        GEMM1 gathers its rows through the pull table itself (the
        reference's dispatch_gemm fusion); ``post_tokens`` (the permuted
        copy) is written only with ``write_post_tokens=True`` — the
        reference bench checks ``outputs`` only
        (bench/dispatch_gemm_bench.py:463-487).  ``validate_tables=False``
        skips the once-per-table-version host check of the tables (a
        read-back that synchronizes the stream)."""
        tok = _data(pre_tokens)[:num_local_tokens]
        Rp = int(num_padded_local_tokens)
        E = weights.shape[0]
        pl = _local_tables(s, pre_tokens, pull_dispatch_indices, padded_tokens_per_expert, E, Rp, node_idx, num_nodes,
                           validate_tables)
        if Rp == 0:
            return outputs
        pull = pull_dispatch_indices[:Rp]
        rb_rows = s.buffer("rb_rows", Rp // 128, pull.device)
        ops.moe_tile_rows(pull, rb_rows)
        if write_post_tokens:
            ops.moe_permute(tok, pull, post_tokens[:Rp], tokens_per_src=num_local_tokens)
        ops.moe_grouped_gemm(tok, weights, outputs[:Rp], padded_tokens_per_expert=pl, mode=0, rb_rows=rb_rows,
                             gather_pull=pull, tokens_per_src=num_local_tokens)
        return outputs

    return _module("dispatch_gemm", s, (), moe_dispatch_gemm_fused=moe_dispatch_gemm_fused)


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
                                            use_gather, num_nodes, cross_node_barrier_ptr=0, *,
                                            write_post_tokens=False, validate_tables=True):
        """Dispatch -> GEMM1 + SwiGLU -> GEMM2 -> top-k weighted combine
        (reference include/operators/dispatch_gemm_glu_combine/dispatch_gemm_glu_combine.cuh:307-548).

        Writes act, y_expert and ``y_out.data_`` [num_local_tokens, H] (fp32
        or bf16) = sum over each token's slots of topk_weights[row] *
        y_expert[row], gathered through owner_offset / row_to_slot /
        row_to_owner (the reference's build_gather_indices CSR,
        bench/dispatch_gemm_glu_combine_bench.py:222-293).  GEMM1 gathers its
        rows through the pull table; ``post_tokens`` is written only with
        ``write_post_tokens=True``.  y_out is overwritten, so the reference's
        zeroing before each call is harmless but not needed.  The slot
        inverse and the per-block row counts are derived from the caller's
        tables on every call (two small launches into session-owned
        buffers: the tables may change between calls); the one-GPU layout
        check (every row owned by this GPU, every slot inside the CSR) runs
        once per table version, as a host read-back that synchronizes the
        stream; ``validate_tables=False`` skips it (the slot inversion still
        bounds-checks every slot on the device)."""
        tok = _data(pre_tokens)[:num_local_tokens]
        yo = _data(y_out)
        Rp = int(num_padded_local_tokens)
        T = int(num_local_tokens)
        E = w1.shape[0]
        dev = yo.device
        pl = _local_tables(s, pre_tokens, pull_dispatch_indices, padded_tokens_per_expert, E, Rp, node_idx, num_nodes,
                           validate_tables)
        key = ("csr", str(dev), owner_offset.data_ptr(), owner_offset._version, row_to_owner.data_ptr(),
               row_to_owner._version, row_to_slot.data_ptr(), row_to_slot._version, Rp, T)
        if validate_tables and not s.checked(key):
            owners = row_to_owner[:Rp].cpu().numpy()
            slots = row_to_slot[:Rp].cpu().numpy()
            nslots = int(owner_offset[T].item())
            mine = owners == 0
            bad = None
            if (owners > 0).any():
                bad = "row_to_owner names other GPUs: these gather tables come from a multi-GPU layout"
            elif nslots != int(mine.sum()) or (mine.any() and (slots[mine].min() < 0 or slots[mine].max() >= nslots)):
                bad = "row_to_slot / owner_offset do not describe this GPU's slots"
            if bad:
                s.unchecked(key)
                raise ValueError(bad)
        nslots_cap = Rp  # every slot index is < R <= R_pad on one GPU (checked above)
        slot_to_row = s.buffer("slot_to_row", nslots_cap, dev)
        ops.moe_invert_slots(row_to_slot[:Rp], row_to_owner[:Rp], slot_to_row, owner=0)
        rb_rows = s.buffer("rb_rows", Rp // 128, dev)
        if Rp:
            ops.moe_tile_rows(pull_dispatch_indices[:Rp], rb_rows)
        post = post_tokens[:Rp] if write_post_tokens else None
        if write_post_tokens and Rp:
            ops.moe_permute(tok, pull_dispatch_indices[:Rp], post, tokens_per_src=T)
        ops.moe_ffn_combine(tok, pull_dispatch_indices[:Rp], topk_weights, owner_offset, slot_to_row, w1, w2,
                            post, act[:Rp], y_expert[:Rp], yo[:T], padded_tokens_per_expert=pl, tokens_per_src=T,
                            rb_rows=rb_rows, fuse_dispatch=True)
        return yo

    return _module("dispatch_gemm_glu_combine", s, ("get_barrier_device_ptr",),
                   moe_dispatch_gemm_glu_combine_fused=moe_dispatch_gemm_glu_combine_fused)


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
