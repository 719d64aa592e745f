"""GPU path against the committed known-answer vectors
(tests/golden/known_answers.npz), through the C-ABI: exact for the integer
GEMM and reduce-scatter outputs, the routing tables and the permuted rows;
rel-Frobenius 2e-2 for the bf16 FFN and combine outputs."""
import numpy as np
import pytest
import torch

from mkernel_amd import ops
from oracle.gemm import rel_fro
from test_golden import F, INDEX_KEYS, _bf, moe_inputs

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _say(msg):
    print(msg, flush=True)


def test_gemm_golden(dev):
    _say("golden gemm 256x256x128")
    A, B = _bf(F["gemm_A"]).to(dev), _bf(F["gemm_B"]).to(dev)
    C = ops.gemm(A, B)
    torch.cuda.synchronize()
    assert torch.equal(C.cpu().float(), torch.from_numpy(F["gemm_C"]).float())


@pytest.mark.parametrize("producers", [0, -1])
def test_gemm_rs_golden(dev, producers):
    _say(f"golden gemm_rs producers={producers}")
    world, rank = (int(v) for v in F["rs_world_rank"])
    A, B, peers = _bf(F["rs_A"]).to(dev), _bf(F["rs_B"]).to(dev), _bf(F["rs_peers"]).to(dev)
    M, N = A.shape[0], B.shape[1]
    rows = M // world
    work = torch.zeros((M, N), dtype=torch.bfloat16, device=dev)
    out = torch.zeros((rows, N), dtype=torch.bfloat16, device=dev)
    nfl = (world - 1) * rows // 128
    if producers:
        recv = torch.zeros_like(peers)
        flags = torch.zeros(nfl, dtype=torch.int32, device=dev)
    else:
        recv = peers.clone()
        flags = torch.full((nfl,), 3, dtype=torch.int32, device=dev)
    order = torch.arange(nfl, dtype=torch.int32, device=dev).flip(0).contiguous()
    counters = torch.zeros(nfl, dtype=torch.int32, device=dev)
    ops.gemm_rs(A, B, work, out, peers, recv, world, rank, flags, order, epoch=3, num_producers=producers,
                stage_counters=counters)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu().float(), torch.from_numpy(F["rs_owned"]).float())


def test_moe_golden(dev):
    _say("golden moe index + ffn + combine")
    m = moe_inputs()
    idx = ops.moe_build_indices_dev(torch.from_numpy(m["ids"]).to(dev), torch.from_numpy(m["gates"]).to(dev),
                                    m["e0"], m["n_local"])
    for k in INDEX_KEYS:
        assert np.array_equal(idx[k].cpu().numpy(), F["moe_" + k]), k
    R_pad = idx["R_pad"]
    post = torch.empty((R_pad, m["H"]), dtype=torch.bfloat16, device=dev)
    act = torch.empty((R_pad, m["I"]), dtype=torch.bfloat16, device=dev)
    ye = torch.empty((R_pad, m["H"]), dtype=torch.bfloat16, device=dev)
    y = torch.empty((m["T"], m["H"]), dtype=torch.bfloat16, device=dev)
    ops.moe_ffn_combine(m["tokens"].to(dev), idx["pull_indices"], idx["row_weight"], idx["owner_offset"],
                        idx["slot_to_row"], m["w1"].to(dev), m["w2"].to(dev), post, act, ye, y,
                        rb_expert=idx["rb_expert"], rb_rows=idx["rb_rows"])
    torch.cuda.synchronize()
    assert torch.equal(post.cpu(), _bf(F["moe_post_x2"], 2))
    assert rel_fro(ye.cpu().float(), torch.from_numpy(F["moe_y_expert"])) < TOL
    assert rel_fro(y.cpu().float(), torch.from_numpy(F["moe_y"])) < TOL
