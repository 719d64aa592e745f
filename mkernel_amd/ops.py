"""Torch-tensor front end of libmk (device memory and streams come from torch;
every computation runs in libmk's HIP kernels through the C-ABI).

All functions launch on torch's current HIP stream and return immediately.
Shape/argument problems raise :class:`mkernel_amd.capi.MkError`.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import capi
from .capi import (AgGemmArgs, GemmAr2Args, GemmArArgs, GemmArgs, GemmRsArgs, MoeCombineArgs, MoeFfnArgs, MoeGroupedGemmArgs,
                   MoeIndex, MoeIndexDevArgs, MoePermuteArgs)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _bf16(t: torch.Tensor, name: str) -> None:
    if t.dtype != torch.bfloat16 or not t.is_cuda or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous bf16 device tensor")


def cu_count() -> int:
    return int(capi.lib().mk_device_cu_count())


_split_ws: dict = {}


def split_workspace(device=None, stream=None) -> torch.Tensor:
    """The K-split workspace the GEMM entry points use by default: one per
    (device, stream), mk_query_workspace_bytes() bytes, zero-filled once
    (every launch leaves it zeroed).  Launches on one stream are ordered, so
    they can share it; launches on different streams get different ones.
    ``stream``: a torch stream, default the current stream of the device.
    Graph capture runs on a stream of its own: fetch the workspace before
    capturing and pass it as ``split_ws``; one first created inside the
    capture has its zero-fill recorded into the graph (about 11 us per
    replay on MI355X).  Every distinct (device, stream handle) keeps its
    workspace (mk_query_workspace_bytes() bytes, ~67 MB on 256 CUs) until
    the process exits or release_split_workspaces() is called; a stream
    created later with a recycled handle reuses that entry, which is safe
    because each launch leaves the workspace zeroed."""
    dev = torch.device("cuda", torch.cuda.current_device() if device is None else torch.device(device).index or 0)
    if stream is None:
        stream = torch.cuda.current_stream(dev)
    key = (dev, stream.cuda_stream)
    ws = _split_ws.get(key)
    if ws is None:
        n = int(capi.lib().mk_query_workspace_bytes(0, 0, 0, 0))
        if n < 0:
            raise capi.MkError("mk_query_workspace_bytes", n, capi.lib().mk_last_error_string().decode())
        ws = torch.zeros(n, dtype=torch.uint8, device=dev)
        _split_ws[key] = ws
    return ws


def release_split_workspaces() -> None:
    """Free every cached default K-split workspace (after synchronizing
    every device that has one, so no queued launch still uses them)."""
    for dev in {k[0] for k in _split_ws}:
        torch.cuda.synchronize(dev)
    _split_ws.clear()


def _ws(split_ws, device) -> tuple:
    """(pointer, bytes) of the K-split workspace: the default one of the
    device's current stream, an explicit tensor, or none at all when
    split_ws is False."""
    if split_ws is False:
        return None, 0
    ws = split_workspace(device) if split_ws is None or split_ws is True else split_ws
    return ws.data_ptr(), ws.numel() * ws.element_size()


def gemm(A: torch.Tensor, B: torch.Tensor, out: torch.Tensor | None = None, num_cus: int = 0,
         tile_m: int = 0, waves: int = 0, split_ws=None) -> torch.Tensor:
    """C = A @ B (bf16 in, fp32 accumulate, bf16 out).  split_ws: None = the
    default per-device K-split workspace, False = no K-split, or a tensor."""
    _bf16(A, "A"); _bf16(B, "B")
    M, K = A.shape
    N = B.shape[1]
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=A.device)
    _bf16(out, "C")
    capi.call("mk_gemm", GemmArgs(_ptr(A), _ptr(B), _ptr(out), M, N, K, K, N, N, num_cus, tile_m, waves,
                                  *_ws(split_ws, A.device)), _stream())
    return out


def ag_gemm(A_shards, A_full, B, C_out, flags, stage_order, epoch: int, gated: bool = True,
            num_producers: int = -1, num_cus: int = 0, spin_limit: int = 0, error_word=None,
            stage_counters=None, split_ws=None, epoch_ptr=None, n_present: int = 0) -> torch.Tensor:
    """Flag-gated AllGather+GEMM; see include/mk.h mk_ag_gemm.  epoch_ptr: an
    optional uint32 device word read for the epoch instead of `epoch`
    (advanced by epoch_advance, e.g. inside a recorded graph).  num_producers
    -1 (default) stages cooperatively, the two halves of the grid taking
    turns to copy ahead; -2 stages cooperatively with every workgroup copying
    an even share before every round; -3 .. -6 run a staging kernel of
    (-2 - num_producers) one-wave workgroups per CU beside the GEMM on a
    side stream (the wave-specialised producer role).  All of them need
    stage_counters (int32 [M/128], zeroed once).  n_present: the first n_present blocks of
    stage_order are already in A_full (published, not copied)."""
    _bf16(A_full, "A_full"); _bf16(B, "B"); _bf16(C_out, "C")
    M, K = A_full.shape
    N = B.shape[1]
    args = AgGemmArgs(_ptr(A_shards), _ptr(A_full), _ptr(B), _ptr(C_out), M, N, K, _ptr(flags), _ptr(stage_order),
                      epoch, int(gated), num_producers, num_cus, spin_limit, _ptr(error_word), _ptr(stage_counters),
                      *_ws(split_ws, A_full.device), _ptr(epoch_ptr), n_present)
    capi.call("mk_ag_gemm", args, _stream())
    return C_out


def gemm_rs(A, B, workspace, output, peer_src, peer_recv, world: int, rank: int, flags, stage_order, epoch: int,
            gated: bool = True, num_producers: int = -1, num_cus: int = 0, spin_limit: int = 0,
            error_word=None, stage_counters=None, split_ws=None, epoch_ptr=None) -> torch.Tensor:
    """GEMM with the reduce-scatter fold in the epilogue; see mk_gemm_rs.
    epoch_ptr: as in ag_gemm."""
    _bf16(A, "A"); _bf16(B, "B")
    M, K = A.shape
    N = B.shape[1]
    args = GemmRsArgs(_ptr(A), _ptr(B), _ptr(workspace), _ptr(output), _ptr(peer_src), _ptr(peer_recv), M, N, K,
                      world, rank, _ptr(flags), _ptr(stage_order), epoch, int(gated), num_producers, num_cus,
                      spin_limit, _ptr(error_word), _ptr(stage_counters), *_ws(split_ws, A.device), _ptr(epoch_ptr))
    capi.call("mk_gemm_rs", args, _stream())
    return output


def gemm_ar(A, B, C_final, peer_src, peer_recv, world: int, flags, stage_order, epoch: int, gated: bool = True,
            num_producers: int = -1, num_cus: int = 0, spin_limit: int = 0, error_word=None, stage_counters=None,
            done_flags=None, split_ws=None, epoch_ptr=None) -> torch.Tensor:
    """GEMM + all-reduce at one rank's share (mk_gemm_ar): C_final = A @ B +
    sum of the world-1 staged peer partials [world-1, M, N], fp32 adds."""
    _bf16(A, "A"); _bf16(B, "B"); _bf16(C_final, "C_final")
    M, K = A.shape
    N = B.shape[1]
    args = GemmArArgs(_ptr(A), _ptr(B), _ptr(C_final), _ptr(peer_src), _ptr(peer_recv), M, N, K, world, _ptr(flags),
                      _ptr(stage_order), epoch, int(gated), num_producers, num_cus, spin_limit, _ptr(error_word),
                      _ptr(stage_counters), _ptr(done_flags), *_ws(split_ws, A.device), _ptr(epoch_ptr))
    capi.call("mk_gemm_ar", args, _stream())
    return C_final


def gemm_ar_two_shot(A, B, C_final, sends, peer_src, peer_recv, peer_reduced, world: int, rank: int, flags,
                     stage_order, epoch: int, gated: bool = True, num_producers: int = -1, num_cus: int = 0,
                     spin_limit: int = 0, error_word=None, stage_counters=None, done_flags=None, split_ws=None,
                     epoch_ptr=None) -> torch.Tensor:
    """GEMM + all-reduce at one rank's share, two-shot (mk_gemm_ar_two_shot):
    this rank's slice of C_final = A @ B + the world-1 staged peer partials
    of that slice ([world-1, M/world, N]); the other slices are the peers'
    reduced rows ``peer_reduced`` ([world-1, M/world, N], slice order
    without ``rank``), staged in; ``sends`` gets this rank's partial rows of
    the other slices.  flags / stage_counters / stage_order cover
    2*(world-1)*(M/world)/128 blocks (partials first, then reduced rows)."""
    _bf16(A, "A"); _bf16(B, "B"); _bf16(C_final, "C_final"); _bf16(sends, "sends")
    M, K = A.shape
    N = B.shape[1]
    args = GemmAr2Args(_ptr(A), _ptr(B), _ptr(C_final), _ptr(sends), _ptr(peer_src), _ptr(peer_recv),
                       _ptr(peer_reduced), M, N, K, world, rank, _ptr(flags), _ptr(stage_order), epoch, int(gated),
                       num_producers, num_cus, spin_limit, _ptr(error_word), _ptr(stage_counters), _ptr(done_flags),
                       *_ws(split_ws, A.device), _ptr(epoch_ptr))
    capi.call("mk_gemm_ar_two_shot", args, _stream())
    return C_final


def epoch_advance(epoch_word: torch.Tensor) -> torch.Tensor:
    """*epoch_word += 1 on the current stream, skipping 0 (mk_epoch_advance);
    epoch_word: a one-element int32/uint32 device tensor."""
    if not epoch_word.is_cuda or epoch_word.numel() != 1 or epoch_word.element_size() != 4:
        raise ValueError("epoch_word must be a one-element 32-bit device tensor")
    capi.check("mk_epoch_advance", capi.lib().mk_epoch_advance(_ptr(epoch_word), C.c_void_p(_stream() or None)))
    return epoch_word


def moe_build_indices(topk_ids: np.ndarray, gates: np.ndarray, e0: int, n_local: int,
                      row_block: int = capi.ROW_BLOCK) -> dict:
    """Host-side routing index build (libmk C++); returns numpy arrays."""
    ids = np.ascontiguousarray(topk_ids, dtype=np.int32)
    g = np.ascontiguousarray(gates, dtype=np.float32)
    T, k = ids.shape
    L = capi.lib()
    R, Rp = C.c_int64(), C.c_int64()
    p = lambda a: a.ctypes.data_as(C.c_void_p)
    capi.check("mk_moe_index_sizes", L.mk_moe_index_sizes(p(ids), T, k, e0, n_local, row_block, C.byref(R), C.byref(Rp)))
    R, Rp = R.value, Rp.value
    o = {
        "padded_tokens_per_expert": np.zeros(n_local, np.int32),
        "local_rb_per_expert": np.zeros(n_local, np.int32),
        "pull_indices": np.zeros((Rp, 3), np.int32),
        "row_expert": np.zeros(Rp, np.int32),
        "rb_expert": np.zeros(Rp // row_block, np.int32),
        "rb_rows": np.zeros(Rp // row_block, np.int32),
        "row_weight": np.zeros(Rp, np.float32),
        "owner_offset": np.zeros(T + 1, np.int32),
        "row_to_slot": np.zeros(Rp, np.int32),
        "row_to_owner": np.zeros(Rp, np.int32),
        "slot_to_row": np.zeros(max(R, 1), np.int32),
    }
    idx = MoeIndex(*[p(o[f]) for f, _ in MoeIndex._fields_])
    capi.check("mk_moe_build_indices", L.mk_moe_build_indices(p(ids), p(g), T, k, e0, n_local, row_block, C.byref(idx)))
    o["slot_to_row"] = o["slot_to_row"][:R]
    o["R"], o["R_pad"] = R, Rp
    return o


_INDEX_TABLES = ("padded_tokens_per_expert", "local_rb_per_expert", "pull_indices", "row_expert", "rb_expert",
                 "rb_rows", "row_weight", "owner_offset", "row_to_slot", "row_to_owner", "slot_to_row")


def moe_build_indices_dev(topk_ids: torch.Tensor, gates: torch.Tensor, e0: int, n_local: int,
                          row_block: int = capi.ROW_BLOCK, sync: bool = True) -> dict:
    """Routing index build on the GPU (mk_moe_build_indices_dev) from device
    top-k ids (int32) and gates (float32) [T, k].  Tables are allocated at
    the worst-case capacity; with sync=True the sizes are read back and the
    returned tensors are views trimmed to R / R_pad rows (the same dict
    layout as moe_build_indices, as device tensors).  With sync=False nothing
    is read back: the tables stay at their capacity and "sizes" holds the
    device int64 {R, R_pad} for moe_ffn_combine(..., sizes=...)."""
    if topk_ids.dtype != torch.int32 or gates.dtype != torch.float32 or not topk_ids.is_cuda:
        raise ValueError("topk_ids must be int32 and gates float32 device tensors")
    ids = topk_ids.contiguous()
    g = gates.contiguous()
    T, k = ids.shape
    dev = ids.device
    # worst case, rounded to whole row blocks so the capacity is a valid
    # row count for the grouped GEMMs
    cap = (T * k + n_local * (row_block - 1) + row_block - 1) // row_block * row_block
    i32 = dict(dtype=torch.int32, device=dev)
    t = {
        "padded_tokens_per_expert": torch.empty(n_local, **i32),
        "local_rb_per_expert": torch.empty(n_local, **i32),
        "pull_indices": torch.empty((cap, 3), **i32),
        "row_expert": torch.empty(cap, **i32),
        "rb_expert": torch.empty((cap + row_block - 1) // row_block, **i32),
        "rb_rows": torch.empty((cap + row_block - 1) // row_block, **i32),
        "row_weight": torch.empty(cap, dtype=torch.float32, device=dev),
        "owner_offset": torch.empty(T + 1, **i32),
        "row_to_slot": torch.empty(cap, **i32),
        "row_to_owner": torch.empty(cap, **i32),
        "slot_to_row": torch.empty(max(cap, 1), **i32),
    }
    L = capi.lib()
    wsb = int(L.mk_moe_index_workspace_bytes(T, k, n_local))
    ws = torch.empty(max(wsb, 4), dtype=torch.uint8, device=dev)
    sizes = torch.zeros(2, dtype=torch.int64, device=dev)
    idx = MoeIndex(*[_ptr(t[f]) for f, _ in MoeIndex._fields_])
    args = MoeIndexDevArgs(_ptr(ids), _ptr(g), T, k, e0, n_local, row_block, cap, _ptr(ws), wsb, _ptr(sizes), idx)
    capi.call("mk_moe_build_indices_dev", args, _stream())
    if not sync:
        t["sizes"] = sizes
        return t
    R, Rp = (int(v) for v in sizes.cpu())
    for f in ("pull_indices", "row_expert", "row_weight", "row_to_slot", "row_to_owner"):
        t[f] = t[f][:Rp]
    t["rb_expert"] = t["rb_expert"][:Rp // row_block]
    t["rb_rows"] = t["rb_rows"][:Rp // row_block]
    t["slot_to_row"] = t["slot_to_row"][:R]
    t["R"], t["R_pad"] = R, Rp
    return t


def moe_permute(tokens, pull, post, tokens_per_src: int | None = None, devs_per_node: int = 1, sizes=None):
    """sizes: optional device int64 {R, R_pad}; post's rows are then a
    capacity and rows past R_pad are skipped."""
    _bf16(tokens, "tokens"); _bf16(post, "post_tokens")
    R_pad, H = post.shape
    tps = tokens.shape[0] if tokens_per_src is None else tokens_per_src
    capi.call("mk_moe_permute", MoePermuteArgs(_ptr(tokens), _ptr(pull), _ptr(post), R_pad, H, tokens.shape[0], tps,
                                                devs_per_node, _ptr(sizes)), _stream())
    return post


def moe_grouped_gemm(A, W, out, rb_expert=None, padded_tokens_per_expert=None, mode: int = 0, num_cus: int = 0,
                     rb_rows=None, split_ws=None, gather_pull=None, tokens_per_src: int | None = None,
                     devs_per_node: int = 1, tile_n: int = 0, sizes=None):
    """mode 0: out = A @ W[e]; mode 1: out = silu(h[:, :I]) * h[:, I:], h = A @ W[e].
    tile_n: output tile width 256 or 512 (0: the library's choice).  sizes:
    optional device int64 {R, R_pad}; the row count is then a capacity and
    row tiles past R_pad are not computed."""
    _bf16(A, "A"); _bf16(W, "W"); _bf16(out, "out")
    # with gather_pull, A is the token buffer and the rows come from the pull table
    R_pad = gather_pull.shape[0] if gather_pull is not None else A.shape[0]
    K = A.shape[1]
    E, _, Nw = W.shape
    tps = A.shape[0] if tokens_per_src is None else tokens_per_src
    args = MoeGroupedGemmArgs(_ptr(A), _ptr(W), _ptr(out), _ptr(rb_expert), _ptr(padded_tokens_per_expert),
                              _ptr(rb_rows), R_pad, K, Nw, E, mode, num_cus, *_ws(split_ws, A.device),
                              _ptr(gather_pull), A.shape[0], tps, devs_per_node, tile_n, _ptr(sizes))
    capi.call("mk_moe_grouped_gemm", args, _stream())
    return out


def moe_tile_rows(pull, rb_rows):
    """rb_rows[b] = real rows in row block b (from the pull table)."""
    capi.check("mk_moe_tile_rows", capi.lib().mk_moe_tile_rows(_ptr(pull), pull.shape[0], _ptr(rb_rows),
                                                               C.c_void_p(_stream() or None)))
    return rb_rows


def moe_invert_slots(row_to_slot, row_to_owner, slot_to_row, owner: int = 0, error_word=None):
    """slot_to_row[:] = -1, then slot_to_row[row_to_slot[r]] = r for the rows
    of `owner` (mk_moe_invert_slots); slots past slot_to_row's length set
    bit 1 of error_word."""
    capi.check("mk_moe_invert_slots", capi.lib().mk_moe_invert_slots(
        _ptr(row_to_slot), _ptr(row_to_owner), row_to_slot.numel(), owner, slot_to_row.numel(), _ptr(slot_to_row),
        _ptr(error_word), C.c_void_p(_stream() or None)))
    return slot_to_row


def moe_combine(y_expert, row_weight, owner_offset, slot_to_row, y_out):
    _bf16(y_expert, "y_expert")
    T, H = y_out.shape
    od = 0 if y_out.dtype == torch.float32 else 1
    if od == 1 and y_out.dtype != torch.bfloat16:
        raise ValueError("y_out must be float32 or bfloat16")
    capi.call("mk_moe_combine", MoeCombineArgs(_ptr(y_expert), _ptr(row_weight), _ptr(owner_offset), _ptr(slot_to_row),
                                                _ptr(y_out), T, H, od), _stream())
    return y_out


def moe_ffn_combine(tokens, pull, row_weight, owner_offset, slot_to_row, w1, w2, post, act, y_expert, y_out,
                    rb_expert=None, padded_tokens_per_expert=None, tokens_per_src: int | None = None,
                    devs_per_node: int = 1, num_cus: int = 0, rb_rows=None, split_ws=None,
                    fuse_dispatch: bool = False, tile_n: int = 0, sizes=None):
    """permute -> grouped GEMM1 + SwiGLU -> grouped GEMM2 -> combine.  With
    fuse_dispatch, GEMM1 reads the token rows through the pull table itself
    (no permute kernel, post may be None and is not written).  sizes: the
    device {R, R_pad} of moe_build_indices_dev(sync=False); the tables and
    buffers are then at their capacity and nothing is read back to the host
    (the call can be recorded in a CUDA/HIP graph)."""
    T, H = y_out.shape
    E, _, I2 = w1.shape
    R_pad = pull.shape[0]
    od = 0 if y_out.dtype == torch.float32 else 1
    tps = tokens.shape[0] if tokens_per_src is None else tokens_per_src
    args = MoeFfnArgs(_ptr(tokens), _ptr(pull), _ptr(rb_expert), _ptr(padded_tokens_per_expert), _ptr(rb_rows),
                      _ptr(row_weight),
                      _ptr(owner_offset), _ptr(slot_to_row), _ptr(w1), _ptr(w2), _ptr(post), _ptr(act), _ptr(y_expert),
                      _ptr(y_out), T, tokens.shape[0], R_pad, H, I2 // 2, E, tps, devs_per_node, od, num_cus,
                      *_ws(split_ws, tokens.device), int(fuse_dispatch), tile_n, _ptr(sizes))
    capi.call("mk_moe_ffn_combine", args, _stream())
    return y_out


def probe_mfma_ceiling(iters: int = 20000, num_wg: int = 0, reps: int = 3) -> dict:
    """MFMA throughput ceiling of the current device under sustained load
    (mk_probe_mfma_ceiling): one 8-wave workgroup per CU issuing independent
    32x32x16 bf16 MFMAs on random operands, no memory traffic.  Returns the
    median TFLOP/s over `reps` launches (HIP events on the launch stream) and
    the engine clock those launches ran at (shader cycles / 100 MHz ticks)."""
    L = capi.lib()
    n_wg = num_wg or cu_count()
    threads = int(L.mk_probe_threads())
    sink = torch.empty(n_wg * threads, dtype=torch.float32, device="cuda")
    clocks = torch.zeros(n_wg * 2, dtype=torch.int64, device="cuda")
    flops = float(n_wg) * (threads // 64) * iters * 16 * 2 * 32 * 32 * 16
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    capi.check("mk_probe_mfma_ceiling", L.mk_probe_mfma_ceiling(iters // 10, n_wg, _ptr(sink), _ptr(clocks), _stream()))
    res = []
    for _ in range(reps):
        s.record()
        capi.check("mk_probe_mfma_ceiling", L.mk_probe_mfma_ceiling(iters, n_wg, _ptr(sink), _ptr(clocks), _stream()))
        e.record()
        torch.cuda.synchronize()
        ck = clocks.view(n_wg, 2).cpu().double()
        ghz = float((ck[:, 0] / ck[:, 1]).median()) * 0.1
        res.append((s.elapsed_time(e), ghz))
    ms, ghz = sorted(res)[len(res) // 2]
    return {"tflops": flops / ms / 1e9, "sclk_ghz": ghz, "workgroups": n_wg, "us": ms * 1e3,
            "finite": bool(torch.isfinite(sink).all())}
