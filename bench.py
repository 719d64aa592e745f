#!/usr/bin/env python3
"""Benchmark of libmk's hot path on one MI355X.

Headline workload (the `value`): BASELINE config 2 — one TP=8 rank's share of
the flag-gated AllGather+GEMM (A_full 16384x8192 assembled from 8 row shards
by the in-launch producer role, 128-row flags published in a seeded random
order, B 8192x3584, C 16384x3584, bf16 in / fp32 accumulate / bf16 out).  A
step is one mk_ag_gemm launch; inputs are resident in HBM before timing.

The same run also reports (under "extra") the ungated GEMM on the same shape
(the gating overhead), config 1 (4096^3), config 3 (GEMM + reduce-scatter
epilogue), config 4 (MoE permute + grouped GEMM1) and config 5 (the full MoE
FFN + combine layer, tokens/s).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload all|ag|...]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import numpy as np
import torch

from mkernel_amd import ops, workloads as wl

METRIC = "fused-GEMM TFLOP/s & % bf16 MFMA peak (1×MI355X); MoE layer tokens/s"
PEAK_BF16_TFLOPS = 2500.0   # MI355X published dense bf16 MFMA peak
PEAK_HBM_GBS = 8000.0       # MI355X published HBM3E bandwidth


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class Timer:
    """HIP events on torch's current stream — the stream libmk launches on."""

    def __init__(self):
        self.s = torch.cuda.Event(enable_timing=True)
        self.e = torch.cuda.Event(enable_timing=True)

    def run(self, fn, steps: int, warmup: int, primed: bool = False) -> float:
        """Mean ms per step of `steps` launches.  primed=False: synchronize
        after the warmup, so the timed region starts with an empty queue and
        the first launch's host latency is inside it (the contract's
        synchronize-bracketed step).  primed=True: the start event is queued
        behind the warmup launches, so the region holds back-to-back launches
        only (steady state, comparable with a profiler's kernel average)."""
        for i in range(warmup):
            fn(i)
        if not primed:
            torch.cuda.synchronize()
        self.s.record()
        for i in range(steps):
            fn(warmup + i)
        self.e.record()
        torch.cuda.synchronize()
        return self.s.elapsed_time(self.e) / steps  # ms per step


def interleaved(variants: dict, steps: int, warmup: int, rounds: int = 3) -> dict:
    """Time several variants of one workload in alternating rounds (the GPU's
    clock and power state drift over a run, so back-to-back blocks of one
    variant bias the comparison); returns the median ms per step of each."""
    t = Timer()
    res = {k: [] for k in variants}
    for r in range(rounds):
        for k, fn in variants.items():
            res[k].append(t.run(fn, steps, warmup if r == 0 else 1))
    return {k: statistics.median(v) for k, v in res.items()}


# --------------------------------------------------------------- workloads
def bench_ag(steps, warmup, producers, extra):
    cfg = wl.AgCfg()
    dev = "cuda"
    A, B, order = wl.ag_inputs(cfg, device=dev)
    A_full = torch.zeros_like(A)
    C = torch.empty((cfg.M, cfg.N), dtype=torch.bfloat16, device=dev)
    flags = torch.zeros(cfg.M // 128, dtype=torch.int32, device=dev)
    counters = torch.zeros(cfg.M // 128, dtype=torch.int32, device=dev)
    order_d = torch.from_numpy(order).to(dev)
    flops = 2.0 * cfg.M * cfg.N * cfg.K
    epoch = [0]

    def gated(i, prod):
        # every step publishes a new epoch; flags and counters are never reset
        epoch[0] += 1
        ops.ag_gemm(A, A_full, B, C, flags, order_d, epoch=epoch[0], num_producers=prod, stage_counters=counters)

    flags_pub = torch.full_like(flags, 2 ** 30)
    # the reference's call semantics: rank 0's own shard is already in A_full
    # (bench/ag_gemm_bench.py:364-372), so only the 7 peer shards are staged
    own = cfg.shard_rows // 128
    A_own = torch.zeros_like(A)
    A_own[:cfg.shard_rows] = A[:cfg.shard_rows]
    order_own = torch.tensor(list(range(own)) + [int(b) for b in order if int(b) >= own], dtype=torch.int32,
                             device=dev)
    epoch_own = [0]

    def gated_own(i):
        epoch_own[0] += 1
        ops.ag_gemm(A, A_own, B, C, flags_own, order_own, epoch=epoch_own[0], num_producers=producers,
                    stage_counters=counters_own, n_present=own)

    flags_own = torch.zeros_like(flags)
    counters_own = torch.zeros_like(counters)
    r = interleaved({
        "gated": lambda i: gated(i, producers),
        # cooperative staging with every workgroup copying before every round
        "even_share": lambda i: gated(i, -2),
        "dedicated": lambda i: gated(i, 32),
        # one-wave staging workgroups co-resident with a register-capped GEMM
        "coresident": lambda i: gated(i, -3),
        "ungated": lambda i: ops.ag_gemm(None, A_full, B, C, None, None, epoch=1, gated=False, num_producers=0),
        # gated, flags already published (pure gating cost, all CUs computing)
        "preset": lambda i: ops.ag_gemm(None, A_full, B, C, flags_pub, order_d, epoch=2 ** 30, num_producers=0),
        "own_shard_local": gated_own,
        # the vendor library (torch.matmul = hipBLASLt) on the same operands
        "torch_matmul": lambda i: torch.matmul(A_full, B, out=C),
    }, steps, warmup)
    ms_med, ms_dedicated, ms_ungated, ms_preset = r["gated"], r["dedicated"], r["ungated"], r["preset"]
    # the headline: W warmup steps, then exactly K timed steps of the gated
    # launch in one region (its mean launch time is the roofline's basis;
    # these are the last K ag_gemm dispatches of the run)
    ms = Timer().run(lambda i: gated(i, producers), steps, warmup)
    extra["ag_gemm"] = {
        "shape": [cfg.M, cfg.N, cfg.K], "producers": producers,
        "us_gated_producer": ms * 1e3, "us_gated_producer_interleaved_median": ms_med * 1e3,
        "us_ungated": ms_ungated * 1e3, "us_gated_flags_preset": ms_preset * 1e3,
        "us_gated_32_dedicated_producers": ms_dedicated * 1e3,
        "us_gated_even_share_staging": r["even_share"] * 1e3,
        "us_gated_coresident_staging_kernel": r["coresident"] * 1e3,
        "us_torch_matmul_ungated": r["torch_matmul"] * 1e3,
        "tflops_gated_producer": flops / ms / 1e9, "tflops_ungated": flops / ms_ungated / 1e9,
        "gating_overhead_producer": ms_med / ms_ungated - 1.0,
        "gating_overhead_flag_check": ms_preset / ms_ungated - 1.0,
        "staging_bytes": 2 * A.numel() * 2,
        "us_gated_own_shard_local": r["own_shard_local"] * 1e3,
        "gating_overhead_own_shard_local": r["own_shard_local"] / ms_ungated - 1.0,
        "gating_note": "flag_check = the gate alone (flags already published); producer = gate + the in-GPU "
                       "producer copying all 8 shards (537 MB read + written by the compute workgroups between "
                       "tile rounds); own_shard_local = the reference's semantics, 7 shards staged",
    }
    return ms, flops, (A_full, B)


def bench_gemm(steps, warmup, extra):
    cfg = wl.GemmCfg()
    A, B = wl.gemm_inputs(cfg, device="cuda")
    C = torch.empty((cfg.M, cfg.N), dtype=torch.bfloat16, device="cuda")
    flops = 2.0 * cfg.M * cfg.N * cfg.K
    ms = Timer().run(lambda i: ops.gemm(A, B, C), steps, warmup)
    # the same launches with the queue kept full: a profiler's per-kernel
    # average excludes the empty-queue start (one host launch latency) that
    # a synchronize-bracketed region of a ~0.1 ms kernel includes
    ms_primed = Timer().run(lambda i: ops.gemm(A, B, C), max(steps, 50), max(warmup, 5), primed=True)
    # the vendor library on the same data in the same process, interleaved
    # (torch.matmul is hipBLASLt here): a same-box comparison
    rv = interleaved({"mk": lambda i: ops.gemm(A, B, C), "torch": lambda i: torch.matmul(A, B, out=C)}, steps, warmup)
    extra["gemm_4096"] = {"us": ms * 1e3, "tflops": flops / ms / 1e9, "frac_peak": flops / ms / 1e9 / PEAK_BF16_TFLOPS,
                          "us_back_to_back": ms_primed * 1e3, "tflops_back_to_back": flops / ms_primed / 1e9,
                          "us_interleaved": rv["mk"] * 1e3, "us_torch_matmul_interleaved": rv["torch"] * 1e3}


def bench_rs(steps, warmup, producers, extra):
    cfg = wl.RsCfg()
    A, B, peers, order = wl.rs_inputs(cfg, device="cuda")
    rows = cfg.M // cfg.world
    work = torch.empty((cfg.M, cfg.N), dtype=torch.bfloat16, device="cuda")
    out = torch.empty((rows, cfg.N), dtype=torch.bfloat16, device="cuda")
    recv = torch.empty_like(peers)
    flags = torch.zeros((cfg.world - 1) * rows // 128, dtype=torch.int32, device="cuda")
    counters = torch.zeros_like(flags)
    order_d = torch.from_numpy(order).to("cuda")
    flops = 2.0 * cfg.M * cfg.N * cfg.K
    epoch = [0]

    def rs(i):
        epoch[0] += 1  # monotonic: flags and counters are never reset
        ops.gemm_rs(A, B, work, out, peers, recv, cfg.world, cfg.rank, flags, order_d, epoch=epoch[0],
                    num_producers=producers, stage_counters=counters)

    # BASELINE config 3 as written: the 7 partials already in place and their
    # flags already published (no staging copy inside the launch)
    recv_pre = peers.clone()
    flags_pub = torch.full_like(flags, 2 ** 30)
    out_pre = torch.empty_like(out)

    def prestaged(i):
        ops.gemm_rs(A, B, work, out_pre, None, recv_pre, cfg.world, cfg.rank, flags_pub, order_d, epoch=2 ** 30,
                    num_producers=0)

    # the same in-launch staging with the partials arriving row block by row
    # block (every peer's block of owned row 0, then of row 1, ...): the
    # spread schedule folds owned row k in round k as its blocks land
    rbs = rows // 128
    order_rows = torch.tensor([q * rbs + rb for rb in range(rbs) for q in range(cfg.world - 1)], dtype=torch.int32,
                              device="cuda")
    epoch_rows = [0]
    flags_rows = torch.zeros_like(flags)
    counters_rows = torch.zeros_like(flags)

    def rs_rows(i):
        epoch_rows[0] += 1
        ops.gemm_rs(A, B, work, out, peers, recv, cfg.world, cfg.rank, flags_rows, order_rows,
                    epoch=epoch_rows[0], num_producers=producers, stage_counters=counters_rows)

    r = interleaved({"rs": rs, "rs_rows": rs_rows, "prestaged": prestaged, "plain": lambda i: ops.gemm(A, B, work)},
                    steps, warmup)
    ms, ms_plain = r["rs"], r["plain"]
    extra["gemm_rs"] = {"shape": [cfg.M, cfg.N, cfg.K], "producers": producers, "us": ms * 1e3,
                        "tflops": flops / ms / 1e9, "us_plain_gemm_same_shape": ms_plain * 1e3,
                        "us_prestaged": r["prestaged"] * 1e3, "tflops_prestaged": flops / r["prestaged"] / 1e9,
                        "us_staged_row_block_order": r["rs_rows"] * 1e3,
                        "overhead_prestaged": r["prestaged"] / ms_plain - 1.0,
                        "overhead_staged_random_order": ms / ms_plain - 1.0,
                        "overhead_staged_row_block_order": r["rs_rows"] / ms_plain - 1.0,
                        "epilogue_bytes_read": peers.numel() * 2,
                        "note": "us: the 7 peer partials staged into recv inside the launch (cooperative copy "
                                "in a seeded random block order, flags published as blocks land); "
                                "us_staged_row_block_order: the same with the blocks arriving row block by row "
                                "block; us_prestaged: partials already in recv and flags published before the "
                                "launch (BASELINE config 3's pre-staged partials).  Owned row tiles are spread "
                                "one per round in arrival order"}


def bench_ar(steps, warmup, producers, extra):
    """GEMM + all-reduce at one rank's share (no BASELINE config: the config-3
    down-projection at half the rows, 8192x8192x3584, 7 staged full peer
    partials of 8192x8192 bf16 N(0,0.5))."""
    M, N, K, world = 8192, 8192, 3584, 8
    A = wl.randn_bf16((M, K), 60, K ** -0.5, "cuda")
    B = wl.randn_bf16((K, N), 61, K ** -0.5, "cuda")
    peers = wl.randn_bf16((world - 1, M, N), 62, 0.5, "cuda")
    recv = torch.empty_like(peers)
    nflags = (world - 1) * M // 128
    flags = torch.zeros(nflags, dtype=torch.int32, device="cuda")
    counters = torch.zeros_like(flags)
    done = torch.zeros((M // 256) * (N // 256), dtype=torch.int32, device="cuda")
    order = torch.from_numpy(wl.stage_order(nflags, 7)).cuda()
    C = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    epoch = [0]

    def ar(i):
        epoch[0] += 1
        ops.gemm_ar(A, B, C, peers, recv, world, flags, order, epoch=epoch[0], num_producers=producers,
                    stage_counters=counters, done_flags=done)

    # Two-shot: this rank (0) reduces its own 1024-row slice from the 7
    # peers' partials of it and receives the other 7 slices already reduced
    # by their owners (each row reduced once across the node)
    rank, s = 0, M // world
    own = ops.gemm(A, B)
    peer_src = peers[:, rank * s:(rank + 1) * s].contiguous()
    reduced = torch.stack([(own[j * s:(j + 1) * s].float() + peers[:, j * s:(j + 1) * s].float().sum(0))
                           .to(torch.bfloat16) for j in range(world) if j != rank])
    del own
    recv2 = torch.empty_like(peer_src)
    sends = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    nb2 = 2 * (world - 1) * s // 128
    flags2 = torch.zeros(nb2, dtype=torch.int32, device="cuda")
    counters2 = torch.zeros_like(flags2)
    rbs = s // 128
    # arrival: the partial blocks of the own slice row block by row block,
    # then the reduced slices
    order2_rows = torch.tensor([q * rbs + rb for rb in range(rbs) for q in range(world - 1)] +
                               list(range((world - 1) * rbs, nb2)), dtype=torch.int32, device="cuda")
    order2_rand = torch.from_numpy(wl.stage_order(nb2, 8)).cuda()
    epoch2 = [0]

    def ar2(order):
        def f(i):
            epoch2[0] += 1
            ops.gemm_ar_two_shot(A, B, C, sends, peer_src, recv2, reduced, world, rank, flags2, order,
                                 epoch=epoch2[0], num_producers=producers, stage_counters=counters2,
                                 done_flags=done)
        return f

    r = interleaved({"ar": ar, "ar2_rows": ar2(order2_rows), "ar2_rand": ar2(order2_rand),
                     "plain": lambda i: ops.gemm(A, B, C)}, steps, warmup)
    flops = 2.0 * M * N * K
    extra["gemm_ar"] = {"shape": [M, N, K], "us": r["ar"] * 1e3, "tflops": flops / r["ar"] / 1e9,
                        "us_plain_gemm_same_shape": r["plain"] * 1e3, "staged_bytes": peers.numel() * 2,
                        "us_two_shot": r["ar2_rows"] * 1e3, "tflops_two_shot": flops / r["ar2_rows"] / 1e9,
                        "us_two_shot_random_order": r["ar2_rand"] * 1e3,
                        "two_shot_staged_bytes": (peer_src.numel() + reduced.numel()) * 2,
                        "note": "us: one-shot, every row reduced here from the 7 staged full peer partials; "
                                "us_two_shot: this rank reduces its 1024-row slice from the 7 peers' partials of "
                                "it and stages the other 7 slices already reduced by their owners (the per-GPU "
                                "work of a node-wide all-reduce that reduces each row once); partial blocks "
                                "arrive row block by row block, then the reduced slices (random_order: a "
                                "seeded random order over all of them)"}


def moe_setup(cfg: wl.MoeCfg):
    tokens, ids, gates, w1, w2 = wl.moe_inputs(cfg, device="cuda")
    idx = ops.moe_build_indices(ids, gates, cfg.e0, cfg.n_local)
    d = {k: torch.from_numpy(np.ascontiguousarray(v)).cuda() for k, v in idx.items() if isinstance(v, np.ndarray)}
    return tokens, w1, w2, idx, d


def bench_moe(steps, warmup, extra):
    """Configs 4 and 5; returns the layer's inputs (for the CPU baseline)."""
    cfg = wl.MoeCfg()
    tokens, w1, w2, idx, d = moe_setup(cfg)
    R, R_pad = idx["R"], idx["R_pad"]
    post = torch.empty((R_pad, cfg.H), dtype=torch.bfloat16, device="cuda")
    h = torch.empty((R_pad, 2 * cfg.I), dtype=torch.bfloat16, device="cuda")
    act = torch.empty((R_pad, cfg.I), dtype=torch.bfloat16, device="cuda")
    ye = torch.empty((R_pad, cfg.H), dtype=torch.bfloat16, device="cuda")
    y = torch.empty((cfg.tokens, cfg.H), dtype=torch.bfloat16, device="cuda")
    t = Timer()

    def dispatch_gemm_unfused(i):
        ops.moe_permute(tokens, d["pull_indices"], post)
        ops.moe_grouped_gemm(post, w1, h, rb_expert=d["rb_expert"], mode=0, rb_rows=d["rb_rows"])

    # config 4: dispatch fused into GEMM1 (rows gathered through the pull table)
    r4 = interleaved({"fused": lambda i: ops.moe_grouped_gemm(tokens, w1, h, rb_expert=d["rb_expert"], mode=0,
                                                              rb_rows=d["rb_rows"], gather_pull=d["pull_indices"]),
                      "unfused": dispatch_gemm_unfused}, steps, warmup)
    ms4, ms4_unfused = r4["fused"], r4["unfused"]
    ms_perm = t.run(lambda i: ops.moe_permute(tokens, d["pull_indices"], post), steps, warmup)
    # the grouped GEMMs at the library's tile width and at 128 x 256
    rg = interleaved({
        "g1": lambda i: ops.moe_grouped_gemm(post, w1, act, rb_expert=d["rb_expert"], mode=1, rb_rows=d["rb_rows"]),
        "g1_256": lambda i: ops.moe_grouped_gemm(post, w1, act, rb_expert=d["rb_expert"], mode=1,
                                                 rb_rows=d["rb_rows"], tile_n=256),
        "g2": lambda i: ops.moe_grouped_gemm(act, w2, ye, rb_expert=d["rb_expert"], mode=0, rb_rows=d["rb_rows"]),
        "g2_256": lambda i: ops.moe_grouped_gemm(act, w2, ye, rb_expert=d["rb_expert"], mode=0,
                                                 rb_rows=d["rb_rows"], tile_n=256)}, steps, warmup)
    ms_g1, ms_g2 = rg["g1"], rg["g2"]
    ms_comb = t.run(lambda i: ops.moe_combine(ye, d["row_weight"], d["owner_offset"], d["slot_to_row"], y),
                    steps, warmup)
    def ffn(fuse, tile_n=0):
        return lambda i: ops.moe_ffn_combine(tokens, d["pull_indices"], d["row_weight"], d["owner_offset"],
                                             d["slot_to_row"], w1, w2, post, act, ye, y, rb_expert=d["rb_expert"],
                                             rb_rows=d["rb_rows"], fuse_dispatch=fuse, tile_n=tile_n)

    # config 5: the layer with the dispatch fused into GEMM1 (the headline),
    # with the separate permute kernel, and with 128 x 256 expert tiles
    r5 = interleaved({"fused": ffn(True), "unfused": ffn(False), "fused_tile256": ffn(True, 256)}, steps, warmup)
    ms5, ms5_unfused = r5["fused"], r5["unfused"]
    # routing index build on the GPU (tables from device top-k ids / gates)
    ids_np, gates_np = wl.zipf_routing(cfg.tokens, cfg.experts, cfg.topk, cfg.zipf_s, 6)
    ids_d = torch.from_numpy(np.ascontiguousarray(ids_np, np.int32)).cuda()
    gates_d = torch.from_numpy(np.ascontiguousarray(gates_np, np.float32)).cuda()
    ms_idx = t.run(lambda i: ops.moe_build_indices_dev(ids_d, gates_d, cfg.e0, cfg.n_local, sync=False), steps, warmup)
    # the host C++ builder (one thread) for comparison
    ops.moe_build_indices(ids_np, gates_np, cfg.e0, cfg.n_local)
    t0 = time.perf_counter()
    for _ in range(3):
        ops.moe_build_indices(ids_np, gates_np, cfg.e0, cfg.n_local)
    ms_idx_host = (time.perf_counter() - t0) / 3 * 1e3
    # the routed layer from device top-k ids / gates with the row count left
    # on the device (index build + FFN + combine, no host read-back), eager
    # and replayed from a HIP graph recorded once
    T_, k_ = ids_d.shape
    cap = (T_ * k_ + cfg.n_local * 127 + 127) // 128 * 128
    act_c = torch.empty((cap, cfg.I), dtype=torch.bfloat16, device="cuda")
    ye_c = torch.empty((cap, cfg.H), dtype=torch.bfloat16, device="cuda")
    # K-split workspace made outside the capture (its one-time zero-fill must
    # not be recorded into the graph)
    ws_routed = ops.split_workspace()

    def routed_layer(i=0):
        tb = ops.moe_build_indices_dev(ids_d, gates_d, cfg.e0, cfg.n_local, sync=False)
        ops.moe_ffn_combine(tokens, tb["pull_indices"], tb["row_weight"], tb["owner_offset"], tb["slot_to_row"], w1,
                            w2, None, act_c, ye_c, y, rb_expert=tb["rb_expert"], rb_rows=tb["rb_rows"],
                            fuse_dispatch=True, sizes=tb["sizes"], split_ws=ws_routed)

    routed_layer()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        routed_layer()
    r_routed = interleaved({"eager": routed_layer, "graph": lambda i: graph.replay()}, steps, warmup)
    used = idx["padded_tokens_per_expert"] > 0
    w_bytes1 = int(used.sum()) * cfg.H * 2 * cfg.I * 2
    w_bytes2 = int(used.sum()) * cfg.I * cfg.H * 2
    f4 = 2.0 * R * cfg.H * 2 * cfg.I
    f5 = 6.0 * R * cfg.H * cfg.I
    layer_bytes = w_bytes1 + w_bytes2 + 2 * R_pad * cfg.H * 2 * 2 + R_pad * cfg.I * 2 * 2 + cfg.tokens * cfg.H * 4
    extra["moe_dispatch_gemm1"] = {"R": R, "R_pad": R_pad, "experts_used": int(used.sum()), "us": ms4 * 1e3,
                                   "tflops": f4 / ms4 / 1e9, "us_permute_then_gemm1": ms4_unfused * 1e3,
                                   "us_permute": ms_perm * 1e3,
                                   # the R routed rows read once, all R_pad rows written
                                   # (padding rows as zeros); the padding rows are not read
                                   "permute_GBs": (R + R_pad) * cfg.H * 2 / ms_perm / 1e6,
                                   "permute_bytes": (R + R_pad) * cfg.H * 2}
    extra["moe_ffn_combine"] = {"us": ms5 * 1e3, "tokens_per_s": cfg.tokens / ms5 * 1e3, "tflops": f5 / ms5 / 1e9,
                                "us_with_separate_permute": ms5_unfused * 1e3,
                                "us_tile_128x256": r5["fused_tile256"] * 1e3,
                                "us_gemm1_swiglu_tile_128x256": rg["g1_256"] * 1e3,
                                "us_gemm2_tile_128x256": rg["g2_256"] * 1e3,
                                "frac_peak": f5 / ms5 / 1e9 / PEAK_BF16_TFLOPS,
                                "hbm_bound_GBs": layer_bytes / ms5 / 1e6,
                                "us_gemm1_swiglu": ms_g1 * 1e3, "us_gemm2": ms_g2 * 1e3, "us_combine": ms_comb * 1e3,
                                "weight_bytes": w_bytes1 + w_bytes2}
    # HBM roofline of the layer: every used expert's W1 and W2 streamed once
    # is the floor; at R routed rows the layer's intensity (FLOP per byte of
    # that traffic) caps the MFMA fraction far below the published peak
    intensity = f5 / layer_bytes
    ridge = PEAK_BF16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)
    extra["moe_ffn_combine"]["roofline"] = {
        "bound": "hbm", "achieved": (w_bytes1 + w_bytes2) / ms5 / 1e6, "peak": PEAK_HBM_GBS, "unit": "GB/s",
        "frac": (w_bytes1 + w_bytes2) / ms5 / 1e6 / PEAK_HBM_GBS, "basis": "unique expert weight bytes per layer",
        "intensity_flop_per_byte": intensity, "ridge_flop_per_byte": ridge,
        "mfma_frac_cap_at_this_intensity": intensity / ridge,
        "note": "the layer streams 2.8 GB of weights for 6*R*H*I FLOP: at this intensity no kernel can exceed "
                "mfma_frac_cap_at_this_intensity of the bf16 MFMA peak, so the HBM fraction is the bar"}
    extra["moe_index_build"] = {"us_gpu": ms_idx * 1e3, "us_host_cpp_1thread": ms_idx_host * 1e3,
                                "entries": cfg.tokens * cfg.topk}
    extra["moe_routed_layer_device_count"] = {
        "what": "GPU index build + fused-dispatch FFN + combine from device top-k ids/gates, row count kept on the "
                "device (buffers at capacity, no host read-back)",
        "us_eager": r_routed["eager"] * 1e3, "us_graph_replay": r_routed["graph"] * 1e3,
        "tokens_per_s_graph": cfg.tokens / r_routed["graph"] * 1e3, "capacity_rows": cap}
    return tokens, ids_np, gates_np, w1, w2


# ------------------------------------------------------------ CPU baseline
def _timed_reps(fn, budget_s: float, max_reps: int = 1000):
    """Run fn repeatedly (after one untimed call) until budget_s of measured
    time has passed; returns (reps, seconds)."""
    fn()
    reps, total = 0, 0.0
    while total < budget_s and reps < max_reps:
        t0 = time.perf_counter()
        fn()
        total += time.perf_counter() - t0
        reps += 1
    return reps, total


def cpu_baseline_moe(inputs, tokens_per_sample: int = 1024, budget_s: float = 10.0) -> dict:
    """Config 5's layer in float32 torch on the host cores, on a bounded
    sample: the first `tokens_per_sample` tokens of the same routing, their
    routed rows gathered with index_select, per-expert matmul, F.silu(g) * u,
    matmul, gate-weighted index_add_ back to token order, repeated for about
    budget_s seconds.  Tokens/s of the sample (the work scales with the
    routed rows)."""
    import torch.nn.functional as F
    cfg = wl.MoeCfg()
    tokens, ids, gates, w1, w2 = (t.cpu() if torch.is_tensor(t) else t for t in inputs)  # the GPU run's inputs
    T = tokens_per_sample
    idx = ops.moe_build_indices(ids[:T], gates[:T], cfg.e0, cfg.n_local)
    pull = torch.from_numpy(idx["pull_indices"]).long()
    real = pull[:, 0] >= 0
    src = pull[real, 2]
    wts = torch.from_numpy(idx["row_weight"])[real]
    expert = torch.from_numpy(idx["row_expert"]).long()[real]
    x = tokens[:T].float()
    w1f, w2f = w1.float(), w2.float()
    torch.set_num_threads(os.cpu_count() or 1)

    def layer():
        rows = x.index_select(0, src)
        y = torch.zeros((T, cfg.H), dtype=torch.float32)
        for e in torch.unique(expert).tolist():
            sel = torch.nonzero(expert == e).flatten()
            h = rows.index_select(0, sel) @ w1f[e]
            a = F.silu(h[:, :cfg.I]) * h[:, cfg.I:]
            ye = a @ w2f[e]
            y.index_add_(0, src.index_select(0, sel), wts.index_select(0, sel)[:, None] * ye)
        return y

    reps, total = _timed_reps(layer, budget_s)
    t = total / reps
    return {"value": T / t, "unit": "tokens/s", "cores": torch.get_num_threads(), "cpu_count": os.cpu_count(),
            "kind": "port",
            "sample": f"first {T} of 4096 tokens ({int(real.sum())} routed rows), fp32 torch on CPU: index_select, "
                      f"per-expert matmul, F.silu(g)*u, matmul, weighted index_add_; {reps} repetitions, "
                      f"{total:.1f} s of CPU work",
            "seconds": t}


def cpu_baseline(A_full, B, rows: int = 2048, budget_s: float = 10.0):
    """The oracle's float32 torch matmul on the host cores, on a bounded
    sample of the same workload: `rows` rows of A_full (one shard) times B,
    repeated for about budget_s seconds."""
    from oracle.gemm import gemm_ref  # CPU baseline leg only
    torch.set_num_threads(os.cpu_count() or 1)
    a = A_full[:rows].cpu()
    b = B.cpu()
    reps, total = _timed_reps(lambda: gemm_ref(a, b), budget_s)
    flops = 2.0 * rows * b.shape[0] * b.shape[1] * reps
    return {"value": flops / total / 1e12, "unit": "TFLOP/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"A_full[:{rows}] @ B ({rows}x{b.shape[0]}x{b.shape[1]}, one shard, fp32 torch on CPU), "
                      f"{reps} repetitions, {total:.1f} s of CPU work"}


def load_traffic():
    """(bytes, source) of the headline kernel's memory traffic per launch,
    read from profiles/traffic.json (rocprofv3 --pmc: the L2's DRAM-destined
    read requests in 32-byte units and its 64-byte write requests,
    calibrated on a copy kernel; the 256 MB MALL serves part of these reads
    and no counter separates them; not measured in this run: the counters
    need their own profiler runs), or (None, None)."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None, None
    src = "profiles/traffic.json (L2 -> fabric bytes, MALL hits included): " + t.get("source", "rocprofv3 --pmc runs")
    return t.get("ag_gemm_gated_bytes_per_launch"), src


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--producers", type=int, default=-1,
                    help="-1: cooperative staging, halves of the grid alternating; -2: cooperative, every "
                         "workgroup before every round; >0: dedicated producer workgroups")
    ap.add_argument("--workload", default="all", choices=["all", "ag", "gemm", "rs", "ar", "moe", "ceiling", "calib"])
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU's share of the path; runs on more than one GPU are not part of this "
              "build: each config is already one rank's share of an 8-GPU job, measured at its real shape on one GPU", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs an MI355X GPU", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    extra = {}
    W, K = args.warmup, args.steps
    line = None
    if args.workload in ("all", "ag"):
        log("[bench] ag_gemm config 2")
        ms, flops, (A_full, B) = bench_ag(K, W, args.producers, extra)
        tflops = flops / ms / 1e9
        traffic, traffic_src = load_traffic()
        line = {
            "metric": METRIC, "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": K, "warmup": W,
            "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "bf16", "data": "synthetic (seeded N(0,1)/sqrt(K) bf16; seeded random stage order)",
            "config": {"workload": "ag_gemm: one TP=8 rank's share, A_full 16384x8192 (8 staged shards), "
                                   "B 8192x3584, C 16384x3584, 128-row flags, staged in-launch (producer role)",
                       "M": 16384, "N": 3584, "K": 8192, "producers": args.producers, "parallelism": "tp8-rank-share"},
            "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tflops / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
                         "traffic_source": traffic_src},
        }
        if not args.no_cpu:
            log("[bench] cpu baseline")
            line["cpu_baseline"] = cpu_baseline(A_full, B)
        del A_full, B
        torch.cuda.empty_cache()
    if args.workload in ("all", "gemm"):
        log("[bench] gemm config 1")
        bench_gemm(K, W, extra)
    if args.workload in ("all", "rs"):
        log("[bench] gemm_rs config 3")
        bench_rs(K, W, args.producers, extra)
        torch.cuda.empty_cache()
    if args.workload in ("all", "ar"):
        log("[bench] gemm_ar (8192x8192x3584, 7 staged peer partials)")
        bench_ar(K, W, args.producers, extra)
        torch.cuda.empty_cache()
    if args.workload in ("all", "moe"):
        log("[bench] moe configs 4/5")
        moe_in = bench_moe(K, W, extra)
        if not args.no_cpu:
            log("[bench] moe cpu baseline")
            extra["moe_ffn_combine"]["cpu_baseline"] = cpu_baseline_moe(moe_in)
        del moe_in
        torch.cuda.empty_cache()
    if args.workload in ("all", "ceiling"):
        # What the matrix cores sustain on this board (power-limited clock),
        # next to the published peak the roofline is priced against.
        log("[bench] mfma ceiling probe")
        c = ops.probe_mfma_ceiling()
        c["frac_of_published_peak"] = c["tflops"] / PEAK_BF16_TFLOPS
        if line is not None:
            c["headline_frac_of_ceiling"] = line["value"] / c["tflops"]
        extra["mfma_ceiling"] = c
    if args.workload == "calib":
        # HBM-counter calibration: libmk's permute kernel as a plain copy of
        # a known size (identity row map, 256 MiB read + 256 MiB written).
        rows, H = 16384, 8192
        src = torch.ones((rows, H), dtype=torch.bfloat16, device="cuda")
        dst = torch.empty_like(src)
        pull = torch.zeros((rows, 3), dtype=torch.int32, device="cuda")
        pull[:, 2] = torch.arange(rows, dtype=torch.int32, device="cuda")
        ms = Timer().run(lambda i: ops.moe_permute(src, pull, dst), K, W)
        extra["copy_calibration"] = {"bytes_read": rows * H * 2, "bytes_written": rows * H * 2, "us": ms * 1e3,
                                     "GBs": 2 * rows * H * 2 / ms / 1e6}
    if line is None:
        line = {"metric": METRIC, "value": None, "unit": "TFLOP/s", "n_gpus": 1, "steps": K, "warmup": W}
    def rnd(v):
        if isinstance(v, float):
            return round(v, 4)
        if isinstance(v, dict):
            return {k: rnd(x) for k, x in v.items()}
        return v

    line["extra"] = rnd(extra)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
