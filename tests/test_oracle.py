"""CPU checks that pin the oracle itself (closed forms, brute force, special
cases, independent restatements) — no GPU needed."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from mkernel_amd import workloads as wl
from oracle import gemm as og
from oracle import moe as om
from oracle.gemm import gemm_ref, rel_fro
from oracle.cmoe import build_indices_c

GOLDEN = Path(__file__).resolve().parent / "golden"


# ---------------------------------------------------------------- GEMM ----
def test_gemm_ref_matches_bruteforce():
    A = wl.randn_bf16((5, 7), 1)
    B = wl.randn_bf16((7, 3), 2)
    assert torch.allclose(og.gemm_ref(A, B).double(), og.gemm_bruteforce(A, B), rtol=1e-6, atol=1e-6)


def test_gemm_ref_special_cases():
    A = wl.randn_bf16((16, 16), 3)
    I = torch.eye(16, dtype=torch.bfloat16)
    assert torch.equal(og.gemm_ref(A, I), A.float())
    assert torch.equal(og.gemm_ref(I, A), A.float())
    Z = A.clone()
    Z[4] = 0
    assert (og.gemm_ref(Z, A)[4] == 0).all()
    B = wl.randn_bf16((16, 8), 4)
    assert torch.allclose(og.gemm_ref(A, B).T, og.gemm_ref(B.T.contiguous(), A.T.contiguous()), atol=1e-5)


def test_ag_ref_is_gemm_on_gathered_rows():
    shards = [wl.randn_bf16((4, 8), s) for s in range(3)]
    B = wl.randn_bf16((8, 5), 9)
    assert torch.equal(og.ag_gemm_ref(shards, B), og.gemm_ref(torch.cat(shards), B))


def test_rs_ref_known_answer():
    A = wl.randn_bf16((16, 8), 1)
    B = wl.randn_bf16((8, 4), 2)
    world, rank = 4, 1
    P = og.gemm_ref(A, B)
    own = P[4:8]
    peers = torch.stack([own] * (world - 1))
    _, owned = og.gemm_rs_ref(A, B, peers, rank, world)
    assert torch.allclose(owned, own * world, rtol=1e-6, atol=1e-6)
    # zero peers => owned slice of the partial
    _, owned0 = og.gemm_rs_ref(A, B, torch.zeros_like(peers), rank, world)
    assert torch.equal(owned0, own)


def test_rel_fro():
    x = torch.ones(4, 4)
    assert og.rel_fro(x, x) == 0.0
    assert abs(og.rel_fro(1.01 * x, x) - 0.01) < 1e-7


# ----------------------------------------------------------------- MoE ----
def _tiny():
    return json.loads((GOLDEN / "index_tiny.json").read_text())


def test_index_tiny_hand_worked():
    g = _tiny()
    out = om.build_indices_py(g["topk_ids"], g["gates"], g["e0"], g["n_local"], g["row_block"])
    for key, val in g["expected"].items():
        got = out[key]
        got = [list(x) for x in got] if key == "pull_indices" else list(got)
        assert got == val, key


@pytest.mark.parametrize("seed,T,E,k,ep,rank", [(0, 64, 16, 4, 4, 0), (1, 300, 64, 8, 8, 3), (2, 1000, 256, 8, 8, 7)])
def test_index_restatements_agree(seed, T, E, k, ep, rank):
    ids, gates = wl.zipf_routing(T, E, k, 1.1, seed)
    n_local = E // ep
    e0 = rank * n_local
    rb = 16
    py = om.build_indices_py(ids, gates, e0, n_local, rb)
    npv = om.build_indices_np(ids, gates, e0, n_local, rb)
    cv = build_indices_c(ids, gates, e0, n_local, rb)
    for key in ("padded_tokens_per_expert", "pull_indices", "row_expert", "row_weight", "owner_offset",
                "row_to_slot", "row_to_owner", "slot_to_row"):
        a = np.asarray(py[key])
        assert np.array_equal(a, np.asarray(npv[key])), key
        assert np.array_equal(a, np.asarray(cv[key])), key
    assert np.array_equal(np.asarray(py["rb_expert"]), npv["rb_expert"])
    assert np.array_equal(np.asarray(py["rb_rows"]), npv["rb_rows"])
    assert np.array_equal(np.asarray(py["local_rb_per_expert"]), npv["local_rb_per_expert"])


def test_index_invariants():
    ids, gates = wl.zipf_routing(2048, 256, 8, 1.1, 6)
    e0, n_local = 64, 32
    o = om.build_indices_np(ids, gates, e0, n_local)
    pull = o["pull_indices"]
    valid = pull[:, 0] >= 0
    # every local (t, k) appears exactly once
    local = [(t, j) for t in range(ids.shape[0]) for j in range(8) if e0 <= ids[t, j] < e0 + n_local]
    assert valid.sum() == len(local) == o["R"]
    assert sorted(pull[valid, 2].tolist()) == sorted(t for t, _ in local)
    assert (pull[~valid] == -1).all()
    assert (o["padded_tokens_per_expert"] % 128 == 0).all()
    assert o["padded_tokens_per_expert"].sum() == o["R_pad"]
    # rows of one expert: tokens ascending, padding at the tail
    start = 0
    for e, n in enumerate(o["padded_tokens_per_expert"]):
        seg = pull[start:start + n]
        toks = seg[seg[:, 0] >= 0, 2]
        assert (np.diff(toks) > 0).all()
        assert (o["row_expert"][start:start + n] == e).all()
        assert (ids[toks] == e0 + e).any(axis=1).all()
        start += n
    # CSR: histogram sums to R, slots a permutation, gates carried over
    assert o["owner_offset"][-1] == o["R"]
    assert sorted(o["row_to_slot"][valid].tolist()) == list(range(o["R"]))
    for r in np.nonzero(valid)[0][:200]:
        t = pull[r, 2]
        j = list(ids[t]).index(e0 + o["row_expert"][r])
        assert o["row_weight"][r] == gates[t, j]


def test_permute_ref():
    tok = wl.randn_bf16((10, 8), 1)
    pull = np.array([[0, 0, 3], [-1, -1, -1], [0, 0, 9]], np.int32)
    out = om.permute_ref(tok, pull)
    assert torch.equal(out[0], tok[3]) and torch.equal(out[2], tok[9]) and (out[1] == 0).all()


def test_permute_ref_multi_source_hand_example():
    """Flattened sources: 2 nodes x 2 devs x 5 tokens; (1, 0, 2) is row
    (1*2 + 0)*5 + 2 = 12, (0, 1, 4) is row 9."""
    tok = wl.randn_bf16((20, 8), 2)
    pull = np.array([[1, 0, 2], [0, 1, 4], [-1, -1, -1], [1, 1, 0]], np.int32)
    out = om.permute_ref(tok, pull, tokens_per_src=5, devs_per_node=2)
    assert torch.equal(out[0], tok[12]) and torch.equal(out[1], tok[9]) and (out[2] == 0).all()
    assert torch.equal(out[3], tok[15])


def test_silu_identities():
    x = torch.linspace(-20, 20, 401)
    one = torch.ones_like(x)
    s = om.silu_mul(x, one)
    assert torch.allclose(s - om.silu_mul(-x, one), x, atol=1e-5)  # odd part
    assert om.silu_mul(torch.zeros(1), torch.ones(1)).item() == 0.0
    assert torch.allclose(s[-1], x[-1], rtol=1e-6)  # silu(x) -> x
    assert abs(s[0].item()) < 1e-6                  # silu(x) -> 0
    assert torch.allclose(s, torch.nn.functional.silu(x), atol=1e-6)


def test_combine_ref_one_hot_and_linearity():
    T, H = 6, 4
    ye = wl.randn_bf16((4, H), 3)
    pull = np.array([[0, 0, 2], [0, 0, 5], [-1, -1, -1], [0, 0, 2]], np.int32)
    w = np.array([0.5, 2.0, 9.0, 0.25], np.float32)
    y = om.combine_ref(ye, w, pull, T)
    assert torch.allclose(y[5], 2.0 * ye[1].float())
    assert torch.allclose(y[2], 0.5 * ye[0].float() + 0.25 * ye[3].float())
    assert (y[[0, 1, 3, 4]] == 0).all()
    y2 = om.combine_ref(ye, 3 * w, pull, T)
    assert torch.allclose(y2, 3 * y)


def test_zipf_routing_properties():
    ids, gates = wl.zipf_routing(1000, 256, 8, 1.1, 6)
    assert ids.shape == (1000, 8)
    assert all(len(set(r)) == 8 for r in ids.tolist())  # distinct experts per token
    assert np.allclose(gates.sum(1), 1.0, atol=1e-6)
    assert (np.diff(gates, axis=1) <= 1e-7).all()        # top-k in descending logit order
    ids2, gates2 = wl.zipf_routing(1000, 256, 8, 1.1, 6)
    assert np.array_equal(ids, ids2) and np.array_equal(gates, gates2)


def test_gemm_ar_ref_known_answers():
    """All-reduce: zero peers leave the plain GEMM; peers equal to the own
    partial give exactly 8x it (integer operands: every sum is exact)."""
    from oracle.gemm import gemm_ar_ref, gemm_ref
    g = torch.Generator().manual_seed(2)
    A = torch.randint(-2, 3, (64, 32), generator=g).to(torch.bfloat16)
    B = torch.randint(-2, 3, (32, 48), generator=g).to(torch.bfloat16)
    P = gemm_ref(A, B)
    zero = torch.zeros((7, 64, 48), dtype=torch.bfloat16)
    assert torch.equal(gemm_ar_ref(A, B, zero), P)
    same = P.bfloat16()[None].expand(7, -1, -1)
    assert torch.equal(gemm_ar_ref(A, B, same), 8 * P)
    # brute force on a tiny case
    a = torch.tensor([[1.0, 2.0]]).bfloat16(); b = torch.tensor([[3.0], [4.0]]).bfloat16()
    peers = torch.tensor([[[0.5]], [[-2.0]]]).bfloat16()
    assert gemm_ar_ref(a, b, peers).item() == 11.0 + 0.5 - 2.0


def test_grouped_gemm_ref_single_expert_is_gemm():
    """One expert covering every row: the grouped GEMM is the plain GEMM."""
    post = wl.randn_bf16((256, 64), 40, 1.0)
    w = wl.randn_bf16((1, 64, 48), 41, 0.125)
    assert torch.equal(om.grouped_gemm_ref(post, w, [256]), gemm_ref(post, w[0]))


def test_grouped_gemm_ref_selects_each_experts_weights():
    """Expert-tagged weights: W[e] = (e + 1) * I (square), so row r comes out
    as (e(r) + 1) * post[r] exactly — a block routed to the wrong expert, an
    off-by-one expert boundary or a dropped empty expert shows up as a wrong
    multiple.  Experts with zero padded rows are skipped without shifting
    the row ranges of the next ones."""
    H = 16
    padded = [128, 0, 256, 128, 0]
    post = wl.randn_bf16((sum(padded), H), 42, 1.0)
    w = torch.stack([(e + 1) * torch.eye(H) for e in range(len(padded))]).to(torch.bfloat16)
    out = om.grouped_gemm_ref(post, w, padded)
    mult = torch.tensor(sum([[e + 1] * n for e, n in enumerate(padded)], []), dtype=torch.float32)
    assert torch.equal(out, post.float() * mult[:, None])


def _ffn_bruteforce(post, w1, w2, padded, I):
    """Per row, per output column, in Python doubles: expert from the padded
    ranges, h = x @ W1[e], act = silu(h[:I]) * h[I:], y = act @ W2[e]."""
    import math
    x = post.float().tolist()
    W1 = w1.float().tolist()
    W2 = w2.float().tolist()
    bounds = np.cumsum(padded)
    acts, ys = [], []
    for r, xr in enumerate(x):
        e = int(np.searchsorted(bounds, r, side="right"))
        h = [sum(xr[k] * W1[e][k][j] for k in range(len(xr))) for j in range(2 * I)]
        a = [h[j] / (1.0 + math.exp(-h[j])) * h[I + j] for j in range(I)]
        acts.append(a)
        ys.append([sum(a[j] * W2[e][j][c] for j in range(I)) for c in range(len(W2[e][0]))])
    return torch.tensor(acts, dtype=torch.float64), torch.tensor(ys, dtype=torch.float64)


def test_ffn_ref_matches_bruteforce():
    """ffn_ref against a scalar restatement on a tiny two-expert case whose
    pre-activations are O(1) (silu far from linear), both halves of W1
    distinct: a swapped gate/up half, a sign slip in the exponential or the
    wrong expert's W2 misses by far more than the tolerance."""
    H, I = 12, 5
    padded = [3, 0, 4]
    post = wl.randn_bf16((7, H), 43, 1.0)
    w1 = wl.randn_bf16((3, H, 2 * I), 44, 0.6)
    w2 = wl.randn_bf16((3, I, H), 45, 0.6)
    act, y = om.ffn_ref(post, w1, w2, padded, I)
    act_b, y_b = _ffn_bruteforce(post, w1, w2, padded, I)
    assert torch.allclose(act.double(), act_b, rtol=1e-5, atol=1e-5)
    assert torch.allclose(y.double(), y_b, rtol=1e-5, atol=1e-5)
    # the same inputs with the gate and up halves swapped differ markedly
    w1s = torch.cat([w1[:, :, I:], w1[:, :, :I]], 2)
    _, y_s = om.ffn_ref(post, w1s, w2, padded, I)
    assert rel_fro(y_s, y_b) > 0.2
