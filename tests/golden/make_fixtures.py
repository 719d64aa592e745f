"""Writes tests/golden/known_answers.npz: small known-answer vectors for the
hot path, produced by the CPU oracle (oracle/) on hand-shaped inputs.

Run from the repo root: python tests/golden/make_fixtures.py

The reference ships no golden vectors for this path (it checks against torch
on the GPU inside its benches: bench/ag_gemm_bench.py:386-400,
bench/gemm_rs_bench.py:820-867, bench/dispatch_gemm_glu_combine_bench.py:829-911),
so these fixtures are this build's own.  Their inputs are chosen so that most
expected values are exact:
* gemm_*: operands in {-1, 0, 1}, K = 128, so every output is an integer of
  magnitude <= 128, exact in fp32 accumulation and in the bf16 store.
* rs_*: a GEMM+reduce-scatter step (world 4, rank 1) with integer partials;
  the owned output is an exact integer sum.
* moe_*: one rank (experts 2-3 of 8, top-2, 64 tokens, row block 128) with a
  hand-written routing that leaves one expert with more rows than another,
  a token routed to both local experts, and tokens routed to none; index
  tables and the permuted rows are exact, the FFN and combine outputs are
  fp32 (SwiGLU's exponential makes them inexact in bf16).
The file is loaded with numpy.load(allow_pickle=False).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import moe as om  # noqa: E402
from oracle.gemm import gemm_ref, gemm_rs_ref  # noqa: E402

OUT = Path(__file__).resolve().parent / "known_answers.npz"

MOE_T, MOE_H, MOE_I, MOE_E, MOE_K, MOE_EP, MOE_RANK = 64, 256, 128, 8, 2, 4, 1


def moe_routing():
    """Hand-shaped top-2 routing over 8 experts; this rank owns experts 2, 3.
    Tokens t % 4 == 0 go to expert 2 (first choice), t % 4 == 1 to expert 3,
    t % 8 == 2 to both (2 first, 3 second), the rest to experts 0/1/4-7 only."""
    ids = np.zeros((MOE_T, MOE_K), np.int32)
    gates = np.zeros((MOE_T, MOE_K), np.float32)
    for t in range(MOE_T):
        if t % 4 == 0:
            ids[t] = (2, 5 + t % 3)
        elif t % 4 == 1:
            ids[t] = (3, t % 2)
        elif t % 8 == 2:
            ids[t] = (2, 3)
        else:
            ids[t] = (t % 2, 4 + t % 4)
        w0 = 0.5 + (t % 5) / 10.0
        gates[t] = (w0, 1.0 - w0)
    return ids, gates


def ternary(shape, gen, scale=1.0):
    return (torch.randint(-1, 2, shape, generator=gen).float() * scale).to(torch.bfloat16)


def main():
    g = torch.Generator().manual_seed(20)
    f = {}
    # plain GEMM, exact integers
    A = ternary((256, 128), g)
    B = ternary((128, 256), g)
    f["gemm_A"] = A.to(torch.int8).numpy()
    f["gemm_B"] = B.to(torch.int8).numpy()
    f["gemm_C"] = gemm_ref(A, B).to(torch.int16).numpy()
    # GEMM + reduce-scatter, world 4, rank 1: M = 1024 (256 owned rows, the
    # library's row-tile multiple)
    world, rank = 4, 1
    A = ternary((1024, 128), g)
    B = ternary((128, 256), g)
    peers = torch.randint(-3, 4, (world - 1, 256, 256), generator=g).float().to(torch.bfloat16)
    P, owned = gemm_rs_ref(A, B, peers, rank, world)
    f["rs_A"] = A.to(torch.int8).numpy()
    f["rs_B"] = B.to(torch.int8).numpy()
    f["rs_peers"] = peers.to(torch.int8).numpy()
    f["rs_world_rank"] = np.array([world, rank], np.int32)
    f["rs_owned"] = owned.to(torch.int16).numpy()
    # MoE FFN + combine at one rank
    ids, gates = moe_routing()
    n_local = MOE_E // MOE_EP
    e0 = MOE_RANK * n_local
    # tokens and W1 in {-1, 0, 1} / 2 put the gate pre-activations at a few
    # units, where silu is far from linear (a sign slip in its exponential
    # changes the outputs by tens of percent)
    tokens = ternary((MOE_T, MOE_H), g, 1.0 / 2)
    w1 = ternary((n_local, MOE_H, 2 * MOE_I), g, 1.0 / 2)
    w2 = ternary((n_local, MOE_I, MOE_H), g, 1.0 / 16)
    idx = om.build_indices_np(ids, gates, e0, n_local)
    post = om.permute_ref(tokens, idx["pull_indices"])
    _, ye = om.ffn_ref(post, w1, w2, idx["padded_tokens_per_expert"], MOE_I)
    y = om.combine_ref(ye, idx["row_weight"], idx["pull_indices"], MOE_T)
    f["moe_dims"] = np.array([MOE_T, MOE_H, MOE_I, MOE_E, MOE_K, MOE_EP, MOE_RANK], np.int32)
    f["moe_topk_ids"] = ids
    f["moe_gates"] = gates
    # inputs as int8 multiples of 1/2 or 1/16: exact
    f["moe_tokens_x2"] = (tokens.float() * 2).to(torch.int8).numpy()
    f["moe_w1_x2"] = (w1.float() * 2).to(torch.int8).numpy()
    f["moe_w2_x16"] = (w2.float() * 16).to(torch.int8).numpy()
    for k in ("padded_tokens_per_expert", "pull_indices", "row_weight", "owner_offset", "slot_to_row"):
        f["moe_" + k] = np.asarray(idx[k])
    f["moe_post_x2"] = (post.float() * 2).to(torch.int8).numpy()
    f["moe_y_expert"] = ye.numpy().astype(np.float32)
    f["moe_y"] = y.numpy().astype(np.float32)
    np.savez_compressed(OUT, **f)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
