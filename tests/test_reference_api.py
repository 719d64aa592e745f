"""The reference's operator modules by name: argument lists match the
reference's pybind definitions (CPU check), and a reference-style call
sequence produces oracle-correct results (GPU)."""
import inspect

import numpy as np
import pytest
import torch

from mkernel_amd import load_module, workloads as wl

# Argument names in order, as the reference's PYBIND11_MODULE blocks declare
# them (include/operators/*/session.cuh; the glu_combine list follows the
# entry point signature at dispatch_gemm_glu_combine.cuh:307-347).
REF_ARGS = {
    ("ag_gemm", "ag_gemm_multinode"): [
        "A", "B", "C", "barrier", "recv_buf_ptr", "fifo_triggers", "fifo_head", "fifo_tail", "fifo_tail_cache",
        "fifo_capacity", "arrival_flags_ptr", "epoch", "node_idx", "num_comm_sms", "a_half_bytes", "A_recv",
        "active_sms", "num_intra_comm_override", "num_nodes"],
    ("gemm_rs", "gemm_rs_fused"): [
        "A", "B", "workspace", "output", "barrier", "ready", "recv_buf_ptr", "staging_buf_ptr", "fifo_triggers",
        "fifo_head", "fifo_tail", "fifo_tail_cache", "fifo_capacity", "arrival_flags_ptr", "epoch", "node_idx",
        "num_comp_sms", "num_intra_comm", "num_send_sms", "num_reduce_sms", "use_acquire_poll",
        "reduce_poll_sleep_ns", "ready_chunk", "staging", "num_nodes"],
    ("gemm_ar", "gemm_ar_multinode"): [
        "A", "B", "C", "barrier", "C_final", "staging_buf_ptr", "recv_buf_ptr", "fifo_triggers", "fifo_head",
        "fifo_tail", "fifo_tail_cache", "fifo_capacity", "arrival_flags_ptr", "epoch", "node_idx",
        "num_intra_comm_sms", "num_inter_comm_sms", "ar_done_ptr", "num_nodes"],
    ("dispatch_gemm", "moe_dispatch_gemm_fused"): [
        "pre_tokens", "peer_tokens", "copy_ready", "post_tokens", "weights", "outputs", "padded_tokens_per_expert",
        "pull_dispatch_indices", "local_rb_per_expert", "barrier", "sync_barrier", "recv_buf_ptr", "fifo_triggers",
        "fifo_head", "fifo_tail", "fifo_tail_cache", "fifo_capacity", "arrival_flags_ptr", "epoch", "node_idx",
        "num_local_tokens", "num_padded_local_tokens", "num_send_sms", "num_copy_sms", "num_comm_sms_intra",
        "num_nodes"],
    ("dispatch_gemm_glu_combine", "moe_dispatch_gemm_glu_combine_fused"): [
        "pre_tokens", "peer_tokens", "copy_ready", "post_tokens", "w1", "w2", "act", "y_expert", "row_expert",
        "topk_weights", "padded_tokens_per_expert", "pull_dispatch_indices", "local_rb_per_expert", "barrier",
        "sync_barrier", "y_out", "comb_buf", "owner_offset", "row_to_slot", "row_to_owner", "inter_comb_buf",
        "inter_owner_offset", "inter_row_to_slot", "inter_row_to_owner", "use_inter_gather", "recv_buf_ptr",
        "fifo_triggers", "fifo_head", "fifo_tail", "fifo_tail_cache", "fifo_capacity", "arrival_flags_ptr",
        "epoch", "node_idx", "num_local_tokens", "num_padded_local_tokens", "num_send_sms", "num_copy_sms",
        "num_comm_sms_intra", "use_gather", "num_nodes", "cross_node_barrier_ptr"],
}


@pytest.mark.parametrize("mod,fn", sorted(REF_ARGS))
def test_reference_argument_lists(mod, fn):
    m = load_module.load(mod)
    params = list(inspect.signature(getattr(m, fn)).parameters)
    ref = REF_ARGS[(mod, fn)]
    assert params[:len(ref)] == ref
    for name in ("DistBuffer", "create_session", "destroy_session", "set_epoch", "get_fifo_handles",
                 "get_arrival_flags_ptr", "get_recv_buf_ptr"):
        assert hasattr(m, name)
    assert m.get_fifo_handles() == (0, 0, 0, 0, 0)


def test_unknown_module():
    with pytest.raises(RuntimeError):
        load_module.load("ring_attention")


@pytest.mark.gpu
def test_ag_gemm_reference_flow(dev):
    from oracle.gemm import ag_gemm_ref, rel_fro
    mod = load_module.load("ag_gemm")
    cfg = wl.AgCfg(world=8, shard_rows=256, K=512, N=512)
    A, B, order = wl.ag_inputs(cfg)
    Abuf = mod.DistBuffer((cfg.M, cfg.K), dtype=torch.bfloat16, local_rank=0, local_world_size=8)
    Arecv = mod.DistBuffer((cfg.M, cfg.K), dtype=torch.bfloat16, local_rank=0, local_world_size=8)
    Arecv.data_.copy_(A.to(dev))
    barrier = mod.DistBuffer((3, 1024, 1024), dtype=torch.int32, local_rank=0, local_world_size=8)
    C = torch.empty((cfg.M, cfg.N), dtype=torch.bfloat16, device=dev)
    mod.create_session(0, "127.0.0.1", 0, 0, 0, 0, 0, 0, 0)
    fifo = mod.get_fifo_handles()
    for epoch in (1, 2):
        mod.set_epoch(epoch)
        mod.ag_gemm_multinode(Abuf, B.to(dev), C, barrier, mod.get_recv_buf_ptr(), *fifo, mod.get_arrival_flags_ptr(),
                              epoch, 0, 8, 0, Arecv, num_intra_comm_override=4, num_nodes=1,
                              stage_order=torch.from_numpy(order).to(dev))
        torch.cuda.synchronize()
        assert rel_fro(C.float(), ag_gemm_ref(A, B)) < 2e-2
    mod.destroy_session()


@pytest.mark.gpu
def test_gemm_rs_reference_flow(dev):
    from oracle.gemm import gemm_rs_ref, rel_fro
    mod = load_module.load("gemm_rs")
    cfg = wl.RsCfg(world=8, rank=5, M=2048, K=256, N=512)
    A, B, peers, order = wl.rs_inputs(cfg)
    rows = cfg.M // cfg.world
    workspace = mod.DistBuffer((cfg.M, cfg.N), dtype=torch.bfloat16, local_rank=5, local_world_size=8)
    output = mod.DistBuffer((rows, cfg.N), dtype=torch.bfloat16, local_rank=5, local_world_size=8)
    staging = mod.DistBuffer(tuple(peers.shape), dtype=torch.bfloat16, local_rank=5, local_world_size=8)
    staging.data_.copy_(peers.to(dev))
    recv = torch.zeros_like(staging.data_)
    barrier = mod.DistBuffer((64,), dtype=torch.int32, local_rank=5, local_world_size=8)
    ready = torch.zeros(1, dtype=torch.int32, device=dev)
    mod.gemm_rs_fused(A.to(dev), B.to(dev), workspace, output, barrier, ready, recv.data_ptr(), 0, 0, 0, 0, 0, 0, 0,
                      1, 0, 240, 8, 0, 0, 1, 0, None, staging, 1)
    torch.cuda.synchronize()
    P, owned = gemm_rs_ref(A, B, peers, 5, 8)
    assert rel_fro(output.data_.float(), owned) < 2e-2


@pytest.mark.gpu
def test_moe_reference_flows(dev):
    from oracle import moe as om
    from oracle.gemm import rel_fro
    cfg = wl.MoeCfg(tokens=512, H=512, I=256, experts=64, topk=8, ep=8, rank=2)
    tokens, ids, gates, w1, w2 = wl.moe_inputs(cfg)
    idx = load_module.build_routing_indices(ids, gates, rank=2, experts=64, ep=8)
    d = {k: torch.from_numpy(np.ascontiguousarray(v)).to(dev) for k, v in idx.items() if isinstance(v, np.ndarray)}
    R_pad, T = idx["R_pad"], cfg.tokens
    # dispatch + GEMM1
    mod = load_module.load("dispatch_gemm")
    pre = mod.DistBuffer((T, cfg.H), dtype=torch.bfloat16)
    pre.data_.copy_(tokens.to(dev))
    post = torch.zeros((R_pad, cfg.H), dtype=torch.bfloat16, device=dev)
    out = torch.zeros((R_pad, 2 * cfg.I), dtype=torch.bfloat16, device=dev)
    mod.moe_dispatch_gemm_fused(pre, None, None, post, w1.to(dev), out, d["padded_tokens_per_expert"],
                                d["pull_indices"], d["local_rb_per_expert"], None, None, 0, 0, 0, 0, 0, 0, 0, 1, 0,
                                T, R_pad, 0, 0, 0, 1)
    torch.cuda.synchronize()
    post_ref = om.permute_ref(tokens, idx["pull_indices"])
    assert torch.equal(post.cpu(), post_ref)
    assert rel_fro(out.float(), om.grouped_gemm_ref(post_ref, w1, idx["padded_tokens_per_expert"])) < 2e-2
    # full FFN + combine
    mod = load_module.load("dispatch_gemm_glu_combine")
    act = torch.zeros((R_pad, cfg.I), dtype=torch.bfloat16, device=dev)
    ye = torch.zeros((R_pad, cfg.H), dtype=torch.bfloat16, device=dev)
    y_out = mod.DistBuffer((T, cfg.H), dtype=torch.float32)
    mod.moe_dispatch_gemm_glu_combine_fused(
        pre, None, None, post, w1.to(dev), w2.to(dev), act, ye, d["row_expert"], d["row_weight"],
        d["padded_tokens_per_expert"], d["pull_indices"], d["local_rb_per_expert"], None, None, y_out, None,
        d["owner_offset"], d["row_to_slot"], d["row_to_owner"], None, None, None, None, 0, 0, 0, 0, 0, 0, 0, 0, 1, 0,
        T, R_pad, 0, 0, 0, 1, 1)
    torch.cuda.synchronize()
    _, ye_ref = om.ffn_ref(post_ref, w1, w2, idx["padded_tokens_per_expert"], cfg.I)
    y_ref = om.combine_ref(ye_ref, idx["row_weight"], idx["pull_indices"], T)
    assert rel_fro(y_out.data_, y_ref) < 2e-2


@pytest.mark.gpu
def test_gemm_ar_reference_flow(dev):
    """gemm_ar_multinode called the way the reference bench calls it
    (bench/gemm_ar_bench.py:445-470): C_final = all-reduce of the partials."""
    from oracle.gemm import gemm_ar_ref, rel_fro
    mod = load_module.load("gemm_ar")
    M, K, N, world = 1024, 256, 512, 8
    A = wl.randn_bf16((M, K), 50, K ** -0.5)
    B = wl.randn_bf16((K, N), 51, K ** -0.5)
    peers = wl.randn_bf16((world - 1, M, N), 52, 0.5)
    C = mod.DistBuffer((M, N), dtype=torch.bfloat16, local_rank=0, local_world_size=world)
    C_final = mod.DistBuffer((M, N), dtype=torch.bfloat16, local_rank=0, local_world_size=world)
    staging = peers.to(dev)
    recv = torch.zeros_like(staging)
    barrier = mod.DistBuffer(((world - 1) * M // 128,), dtype=torch.int32, local_rank=0, local_world_size=world)
    ar_done = torch.zeros((M // 256) * (N // 256), dtype=torch.int32, device=dev)
    mod.set_epoch(1)
    mod.gemm_ar_multinode(A.to(dev), B.to(dev), C, barrier, C_final, staging.data_ptr(), recv.data_ptr(),
                          0, 0, 0, 0, 0, 0, 1, 0, 4, 0, ar_done.data_ptr(), num_nodes=1)
    torch.cuda.synchronize()
    assert rel_fro(C_final.data_.float(), gemm_ar_ref(A, B, peers)) < 2e-2
    assert (ar_done.cpu() == 1).all()
