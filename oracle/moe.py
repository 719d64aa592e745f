"""CPU restatement of the MoE expert path (test-only).

Routing indices follow the reference's host-side builders for one rank that
owns local experts [e0, e0 + n_local) and receives every token from a single
source (node 0, dev 0):
* build_routing / padded_list      reference bench/dispatch_gemm_bench.py:127-166
* build_pull_indices (LOCAL_FIRST)  reference bench/dispatch_gemm_bench.py:169-188
* build_gather_indices (CSR)        reference bench/dispatch_gemm_glu_combine_bench.py:222-293
* local_rb_per_expert, row_expert   reference bench/dispatch_gemm_glu_combine_bench.py:511-527
The numerics follow the reference's torch checks:
* permute   post_ref[row] = tokens[src]             bench/dispatch_gemm_bench.py:463-470
* FFN       silu(post@w1[:, :I]) * (post@w1[:, I:]) @ w2, fp32
                                                    bench/dispatch_gemm_glu_combine_bench.py:829-848
* combine   y_ref[t] += w_r * y_expert[r]           bench/dispatch_gemm_glu_combine_bench.py:886-911
"""
from __future__ import annotations

import numpy as np
import torch

ROW_BLOCK = 128


def build_indices_py(topk_ids, gates, e0: int, n_local: int, row_block: int = ROW_BLOCK) -> dict:
    """Pure-Python restatement (small inputs). topk_ids/gates: [T][k] lists or arrays."""
    ids = [list(map(int, r)) for r in topk_ids]
    gts = [list(map(float, r)) for r in gates]
    T = len(ids)
    # build_routing: expert -> [(token, k)] in token order
    e2t = [[] for _ in range(n_local)]
    for t in range(T):
        for k, e in enumerate(ids[t]):
            if e0 <= e < e0 + n_local:
                e2t[e - e0].append((t, k))
    padded = [((len(l) + row_block - 1) // row_block) * row_block for l in e2t]
    # build_pull_indices: local expert ascending, padding rows (-1,-1,-1)
    pull, row_expert, row_weight = [], [], []
    for e in range(n_local):
        for i in range(padded[e]):
            if i < len(e2t[e]):
                t, k = e2t[e][i]
                pull.append((0, 0, t))
                row_weight.append(gts[t][k])
            else:
                pull.append((-1, -1, -1))
                row_weight.append(0.0)
            row_expert.append(e)
    # build_gather_indices with one producer / one owner: count, CSR, then
    # slots handed out in row order.
    count = [0] * T
    for (sn, sd, st) in pull:
        if sn >= 0:
            count[st] += 1
    off = [0] * (T + 1)
    for t in range(T):
        off[t + 1] = off[t] + count[t]
    running = [0] * T
    row_to_slot, row_to_owner = [], []
    for (sn, sd, st) in pull:
        if sn < 0:
            row_to_slot.append(0)
            row_to_owner.append(-1)
            continue
        row_to_slot.append(off[st] + running[st])
        running[st] += 1
        row_to_owner.append(sd)
    slot_to_row = [0] * off[T]
    for r, (s, o) in enumerate(zip(row_to_slot, row_to_owner)):
        if o >= 0:
            slot_to_row[s] = r
    rb_rows = [sum(1 for (sn, _, _) in pull[b:b + row_block] if sn >= 0) for b in range(0, len(pull), row_block)]
    return {
        "padded_tokens_per_expert": padded,
        "rb_rows": rb_rows,
        "local_rb_per_expert": [len(l) // row_block for l in e2t],
        "pull_indices": pull,
        "row_expert": row_expert,
        "rb_expert": row_expert[::row_block],
        "row_weight": row_weight,
        "owner_offset": off,
        "row_to_slot": row_to_slot,
        "row_to_owner": row_to_owner,
        "slot_to_row": slot_to_row,
        "R": off[T],
        "R_pad": len(pull),
    }


def build_indices_np(topk_ids: np.ndarray, gates: np.ndarray, e0: int, n_local: int,
                     row_block: int = ROW_BLOCK) -> dict:
    """Vectorised numpy restatement with the same outputs as build_indices_py."""
    topk_ids = np.asarray(topk_ids, dtype=np.int64)
    gates = np.asarray(gates, dtype=np.float32)
    T, k = topk_ids.shape
    flat = topk_ids.reshape(-1) - e0
    tok = np.repeat(np.arange(T), k)
    kk = np.tile(np.arange(k), T)
    sel = (flat >= 0) & (flat < n_local)
    le, lt, lk = flat[sel], tok[sel], kk[sel]
    order = np.lexsort((lk, lt, le))  # by expert, then token, then k
    le, lt, lk = le[order], lt[order], lk[order]
    cnt = np.bincount(le, minlength=n_local)
    padded = (cnt + row_block - 1) // row_block * row_block
    R, R_pad = int(cnt.sum()), int(padded.sum())
    pad_start = np.concatenate([[0], np.cumsum(padded)[:-1]])
    real_start = np.concatenate([[0], np.cumsum(cnt)[:-1]])
    rank_in_e = np.arange(R) - real_start[le]
    rows = pad_start[le] + rank_in_e
    pull = np.full((R_pad, 3), -1, dtype=np.int32)
    pull[rows, 0] = 0
    pull[rows, 1] = 0
    pull[rows, 2] = lt
    row_expert = np.repeat(np.arange(n_local), padded).astype(np.int32)
    row_weight = np.zeros(R_pad, dtype=np.float32)
    row_weight[rows] = gates[lt, lk]
    count = np.bincount(lt, minlength=T)
    off = np.concatenate([[0], np.cumsum(count)]).astype(np.int32)
    # slot = off[t] + (number of earlier rows with the same token)
    o2 = np.lexsort((rows, lt))  # rows grouped by token, ascending row
    st = lt[o2]
    first = np.concatenate([[0], np.cumsum(count)[:-1]])
    within = np.arange(R) - first[st]
    row_to_slot = np.zeros(R_pad, dtype=np.int32)
    row_to_slot[rows[o2]] = off[st] + within
    row_to_owner = np.full(R_pad, -1, dtype=np.int32)
    row_to_owner[rows] = 0
    slot_to_row = np.zeros(R, dtype=np.int32)
    slot_to_row[row_to_slot[rows]] = rows
    rb_rows = (pull[:, 0] >= 0).reshape(-1, row_block).sum(1).astype(np.int32) if R_pad else np.zeros(0, np.int32)
    return {
        "padded_tokens_per_expert": padded.astype(np.int32),
        "rb_rows": rb_rows,
        "local_rb_per_expert": (cnt // row_block).astype(np.int32),
        "pull_indices": pull,
        "row_expert": row_expert,
        "rb_expert": row_expert[::row_block].copy(),
        "row_weight": row_weight,
        "owner_offset": off,
        "row_to_slot": row_to_slot,
        "row_to_owner": row_to_owner,
        "slot_to_row": slot_to_row,
        "R": R,
        "R_pad": R_pad,
    }


def permute_ref(tokens: torch.Tensor, pull: np.ndarray | torch.Tensor, tokens_per_src: int | None = None,
                devs_per_node: int = 1) -> torch.Tensor:
    """post[r] = tokens[src_row(r)] (bit-exact), zero rows for padding.

    With one source (the default) src_row = src_token, as the reference's
    single-rank benches build it.  Several sources are flattened into one
    buffer of tokens_per_src rows each: src_row = (src_node * devs_per_node +
    src_dev) * tokens_per_src + src_token — this build's layout for the
    reference's per-device pre_tokens / peer_tokens views
    (src/dispatch_gemm.cu:125-168)."""
    pull = torch.as_tensor(np.asarray(pull)).long()
    tokens = tokens.cpu()
    out = torch.zeros((pull.shape[0], tokens.shape[1]), dtype=tokens.dtype)
    valid = (pull[:, 0] >= 0) & (pull[:, 2] >= 0)
    if tokens_per_src is None:
        rows = pull[valid, 2]
    else:
        rows = (pull[valid, 0] * devs_per_node + pull[valid, 1]) * tokens_per_src + pull[valid, 2]
    out[valid] = tokens[rows]
    return out


def silu_mul(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    """silu(g) * u = g / (1 + exp(-g)) * u in float32."""
    g = g.float()
    return g / (1.0 + torch.exp(-g)) * u.float()


def grouped_gemm_ref(post: torch.Tensor, w: torch.Tensor, padded) -> torch.Tensor:
    """out[rows_e] = post[rows_e] @ w[e] per local expert, fp32."""
    post = post.cpu().float()
    out = torch.zeros((post.shape[0], w.shape[2]), dtype=torch.float32)
    r = 0
    for e, n in enumerate(list(map(int, padded))):
        if n:
            out[r:r + n] = post[r:r + n] @ w[e].cpu().float()
        r += n
    return out


def ffn_ref(post: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, padded, I: int):
    """Returns (act fp32 [R_pad, I], y_expert fp32 [R_pad, H]); fp32 throughout."""
    h = grouped_gemm_ref(post, w1, padded)
    act = silu_mul(h[:, :I], h[:, I:])
    y = torch.zeros((post.shape[0], w2.shape[2]), dtype=torch.float32)
    r = 0
    for e, n in enumerate(list(map(int, padded))):
        if n:
            y[r:r + n] = act[r:r + n] @ w2[e].cpu().float()
        r += n
    return act, y


def combine_ref(y_expert: torch.Tensor, row_weight, pull, num_tokens: int) -> torch.Tensor:
    """y[t] = sum over rows r with pull[r] = (., ., t) of w[r] * y_expert[r], fp32,
    rows in ascending order (the CSR slot order)."""
    pull = torch.as_tensor(np.asarray(pull)).long()
    w = torch.as_tensor(np.asarray(row_weight), dtype=torch.float32)
    ye = y_expert.cpu().float()
    y = torch.zeros((num_tokens, ye.shape[1]), dtype=torch.float32)
    valid = torch.nonzero(pull[:, 0] >= 0).flatten()
    y.index_add_(0, pull[valid, 2], w[valid, None] * ye[valid])
    return y
