"""The reference's operator modules by name: argument lists match the
reference's pybind definitions, calls the one-GPU build cannot serve are
refused (CPU checks), and the reference benches' own call sequence — reset
the buffers the bench resets, write this rank's data where the bench writes
it, call, check — gives oracle-correct results (GPU)."""
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


# Default values the reference's pybind blocks give (include/operators/
# ag_gemm/session.cuh:227-228, dispatch_gemm_glu_combine/session.cuh:154).
# A required reference argument after defaulted ones (ag_gemm's num_nodes)
# needs a default in Python; it is not listed.
REF_DEFAULTS = {
    ("ag_gemm", "ag_gemm_multinode"): {"active_sms": 132, "num_intra_comm_override": 0},
    ("dispatch_gemm_glu_combine", "moe_dispatch_gemm_glu_combine_fused"): {"cross_node_barrier_ptr": 0},
}


@pytest.mark.parametrize("mod,fn", sorted(REF_DEFAULTS))
def test_reference_argument_defaults(mod, fn):
    sig = inspect.signature(getattr(load_module.load(mod), fn))
    for name, value in REF_DEFAULTS[(mod, fn)].items():
        assert sig.parameters[name].default == value, name
    # every other reference argument before the first defaulted one is required
    ref = REF_ARGS[(mod, fn)]
    first = min(ref.index(n) for n in REF_DEFAULTS[(mod, fn)])
    for name in ref[:first]:
        assert sig.parameters[name].default is inspect.Parameter.empty, name


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



def test_dist_buffer_constructors():
    t = torch.zeros((4, 8), dtype=torch.bfloat16)
    b = load_module.DistBuffer(t, 3, 8)
    assert b.data_ is t and b.data() is t and (b.local_rank_, b.local_world_size_) == (3, 8)
    assert not b.multicast_enabled and b.multicast_ptr_u64 == 0
    with pytest.raises(ValueError):
        load_module.DistBuffer(t, 8, 8)


def _fifo():
    return (0, 0, 0, 0, 0)


def test_emulated_rank_needs_peer_data():
    """local_world_size > 1 on one GPU: without the peers' data the call is
    refused before anything runs (the peers' shards / partials do not exist
    here), and multi-node calls are refused."""
    A = load_module.DistBuffer(torch.zeros((2048, 256), dtype=torch.bfloat16), 2, 8)
    B = torch.zeros((256, 256), dtype=torch.bfloat16)
    C = torch.zeros((2048, 256), dtype=torch.bfloat16)
    ag = load_module.load("ag_gemm")
    with pytest.raises(ValueError, match="peer_shards"):
        ag.ag_gemm_multinode(A, B, C, None, 0, *_fifo(), 0, 1, 0, 8, 0, None, 0, 4, 1)
    with pytest.raises(ValueError, match="num_nodes"):
        ag.ag_gemm_multinode(A, B, C, None, 0, *_fifo(), 0, 1, 0, 8, 0, None, 0, 4, 2)
    rs = load_module.load("gemm_rs")
    out = load_module.DistBuffer(torch.zeros((256, 256), dtype=torch.bfloat16), 5, 8)
    ws = load_module.DistBuffer(torch.zeros((2048, 256), dtype=torch.bfloat16), 5, 8)
    with pytest.raises(ValueError, match="peer_partials"):
        rs.gemm_rs_fused(A.data_, B, ws, out, None, None, 0, 0, *_fifo(), 0, 1, 0, 240, 8, 0, 0, 1, 0, None, None, 1)
    ar = load_module.load("gemm_ar")
    Cd = load_module.DistBuffer(torch.zeros((2048, 256), dtype=torch.bfloat16), 0, 8)
    with pytest.raises(ValueError, match="peer_partials"):
        ar.gemm_ar_multinode(A.data_, B, Cd, None, Cd, 0, 0, *_fifo(), 0, 1, 0, 4, 0, 0, num_nodes=1)


def _glu_call(mod, pre, tables, T, R_pad, H=256, I=128, E=2, node_idx=0):
    w1 = torch.zeros((E, H, 2 * I), dtype=torch.bfloat16)
    w2 = torch.zeros((E, I, H), dtype=torch.bfloat16)
    z = torch.zeros((R_pad, H), dtype=torch.bfloat16)
    act = torch.zeros((R_pad, I), dtype=torch.bfloat16)
    y = torch.zeros((T, H), dtype=torch.float32)
    return mod.moe_dispatch_gemm_glu_combine_fused(
        pre, None, None, z, w1, w2, act, z, tables["row_expert"], tables["row_weight"],
        tables["padded"], tables["pull"], None, None, None, y, None, tables["owner_offset"], tables["row_to_slot"],
        tables["row_to_owner"], None, None, None, None, 0, 0, *_fifo(), 0, 1, node_idx, T, R_pad, 0, 0, 0, 1, 1)


def _multi_gpu_tables(T=4, R_pad=256):
    """Tables as the reference's build_gather_indices writes them for a
    2-GPU node (bench/dispatch_gemm_glu_combine_bench.py:264-279): rows of
    tokens owned by GPU 1 carry row_to_owner 1 and slots in GPU 1's
    comb_buf, which may lie past this GPU's rows."""
    pull = torch.full((R_pad, 3), -1, dtype=torch.int32)
    pull[:4] = torch.tensor([[0, 0, 0], [0, 0, 1], [0, 1, 0], [0, 1, 3]], dtype=torch.int32)
    owner = torch.full((R_pad,), -1, dtype=torch.int32)
    owner[:4] = torch.tensor([0, 0, 1, 1], dtype=torch.int32)
    slot = torch.zeros((R_pad,), dtype=torch.int32)
    slot[:4] = torch.tensor([0, 1, 900, 901], dtype=torch.int32)
    return {"pull": pull, "row_to_owner": owner, "row_to_slot": slot,
            "owner_offset": torch.tensor([0, 1, 2, 2, 2], dtype=torch.int32),
            "padded": torch.tensor([128, 128], dtype=torch.int32), "row_expert": torch.zeros(R_pad, dtype=torch.int32),
            "row_weight": torch.ones(R_pad, dtype=torch.float32)}


def test_moe_refuses_multi_gpu_tables():
    """Gather tables of a multi-GPU layout (rows pulled from, or combined on,
    another GPU; slots in another GPU's comb_buf) are refused before any
    launch: the slot inverse would otherwise index past this GPU's rows."""
    mod = load_module.load("dispatch_gemm_glu_combine")
    t = _multi_gpu_tables()
    pre1 = load_module.DistBuffer(torch.zeros((4, 256), dtype=torch.bfloat16), 0, 1)
    with pytest.raises(ValueError, match="other GPUs"):
        _glu_call(mod, pre1, t, 4, 256)
    pre2 = load_module.DistBuffer(torch.zeros((4, 256), dtype=torch.bfloat16), 0, 2)
    with pytest.raises(ValueError, match="one-process"):
        _glu_call(mod, pre2, t, 4, 256)
    # pull rows local, but the combine tables name GPU 1 as an owner
    t["pull"][2:4, 1] = 0
    with pytest.raises(ValueError, match="row_to_owner"):
        _glu_call(mod, pre1, t, 4, 256)
    # slots past this GPU's CSR
    t["row_to_owner"][2:4] = 0
    t["owner_offset"] = torch.tensor([0, 2, 3, 3, 4], dtype=torch.int32)
    with pytest.raises(ValueError, match="slots"):
        _glu_call(mod, pre1, t, 4, 256)
    with pytest.raises(ValueError, match="padded"):
        t["padded"] = torch.tensor([128, 0, 0], dtype=torch.int32)
        _glu_call(mod, pre1, t, 4, 256)


# ---------------------------------------------------------------- GPU ----
def _say(msg):
    print(f"[case] {msg}", flush=True)


def _ag_reference_flow(dev, world, rank, iters=3):
    from oracle.gemm import ag_gemm_ref, rel_fro
    mod = load_module.load("ag_gemm")
    cfg = wl.AgCfg(world=world, shard_rows=2048 // world, K=512, N=512)
    A, B, order = wl.ag_inputs(cfg)
    M, rows = cfg.M, cfg.shard_rows
    lo, hi = rank * rows, (rank + 1) * rows
    a_tk = mod.DistBuffer((M, cfg.K), torch.bfloat16, rank, world)
    a_recv = mod.DistBuffer((M, cfg.K), torch.bfloat16, rank, world)
    barrier = mod.DistBuffer((2, 1024, 1024), torch.int32, rank, world, True)
    Bd = B.to(dev)
    C = torch.zeros((M, cfg.N), dtype=torch.bfloat16, device=dev)
    # what the peers deliver; this rank's own rows hold junk that must never be read
    peers = A.clone()
    peers[lo:hi] = 7.0
    peers = peers.to(dev)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    mod.create_session(0, "127.0.0.1", 0, 0, 0, 0, 0, 0, 0)
    fifo, arrival, recv = mod.get_fifo_handles(), mod.get_arrival_flags_ptr(), mod.get_recv_buf_ptr()
    assert arrival != 0
    epoch = 1
    mod.set_epoch(epoch)
    ref = ag_gemm_ref(A, B)
    for it in range(iters):
        # reset_state of bench/ag_gemm_bench.py:364-372 (the epoch stays 1 there)
        barrier.data_.zero_()
        a_tk.data_.zero_()
        a_tk.data_[lo:hi].copy_(A[lo:hi].to(dev))
        a_recv.data_.zero_()
        C.zero_()
        kw = {"peer_shards": peers, "stage_order": torch.from_numpy(order).to(dev)} if world > 1 else {}
        mod.ag_gemm_multinode(a_tk, Bd, C, barrier, recv, *fifo, arrival, epoch, 0, 16, rows * cfg.K * 2, a_recv,
                              cus, 16, 1, **kw)
        torch.cuda.synchronize()
        err = rel_fro(C.float(), ref)
        assert err < 2e-2, (it, err)
        assert torch.equal(a_tk.data_.cpu(), A), "gathered A differs from the shards"
        assert (a_recv.data_ == 0).all() and (barrier.data_ == 0).all(), "A_recv / barrier were written"
    mod.destroy_session()


@pytest.mark.gpu
@pytest.mark.parametrize("world,rank", [(1, 0), (8, 3), (8, 0), (4, 3)])
def test_ag_gemm_reference_flow(dev, world, rank):
    """bench/ag_gemm_bench.py:364-384 as a sequence: reset, write the own
    shard into A, call with the bench's positional arguments (active_sms =
    CU count, intra_comm_sms > 0, a fixed epoch), check."""
    _say(f"ag reference flow world={world} rank={rank}")
    _ag_reference_flow(dev, world, rank)


@pytest.mark.gpu
@pytest.mark.parametrize("world,rank", [(1, 0), (8, 5)])
def test_gemm_rs_reference_flow(dev, world, rank):
    """bench/gemm_rs_bench.py:742-766: reset every buffer (staging included),
    advance the epoch, call, check the owned slice."""
    from oracle.gemm import gemm_rs_ref, rel_fro
    _say(f"rs reference flow world={world} rank={rank}")
    mod = load_module.load("gemm_rs")
    cfg = wl.RsCfg(world=max(world, 2), rank=rank, M=2048, K=256, N=512)
    A, B, _, _ = wl.rs_inputs(cfg)
    M, N = cfg.M, cfg.N
    rows = M // world
    workspace = mod.DistBuffer((M, N), torch.bfloat16, rank, world)
    output = mod.DistBuffer((rows, N), torch.bfloat16, rank, world)
    barrier = mod.DistBuffer((2, 1024, 1024), torch.int32, rank, world, True)
    ready = torch.zeros(64, dtype=torch.int32, device=dev)
    ready_chunk = mod.DistBuffer((4096,), torch.int32, rank, world, True)
    staging = mod.DistBuffer((rows, N), torch.bfloat16, rank, world)
    Ad, Bd = A.to(dev), B.to(dev)
    pp = None
    if world > 1:
        pp = wl.randn_bf16((world - 1, rows, N), 33, 0.5).to(dev)
        ref = gemm_rs_ref(A, B, pp.cpu(), rank, world)[1]
    else:
        ref = gemm_rs_ref(A, B, torch.zeros((0, rows, N)), 0, 1)[1]
    fifo = mod.get_fifo_handles()
    epoch = 1
    mod.set_epoch(epoch)
    for it in range(3):
        workspace.data_.zero_(); output.data_.zero_(); ready.zero_()
        barrier.data_.zero_(); ready_chunk.data_.zero_(); staging.data_.zero_()
        mod.zero_recv_buf()
        epoch += 1
        mod.set_epoch(epoch)
        kw = {"peer_partials": pp} if world > 1 else {}
        mod.gemm_rs_fused(Ad, Bd, workspace, output, barrier, ready, mod.get_recv_buf_ptr(),
                          staging.data_.data_ptr(), *fifo, mod.get_arrival_flags_ptr(), epoch, 0,
                          200, 16, 8, 32, True, 0, ready_chunk, staging, num_nodes=1, **kw)
        torch.cuda.synchronize()
        err = rel_fro(output.data_.float(), ref)
        assert err < 2e-2, (it, err)
        assert (staging.data_ == 0).all(), "the reference's accumulation buffer was written"
        if world > 1:
            P = (A.float() @ B.float())
            own = torch.zeros(M, dtype=torch.bool)
            own[rank * rows:(rank + 1) * rows] = True
            assert rel_fro(workspace.data_.float()[~own], P[~own]) < 2e-2  # the would-be sends


@pytest.mark.gpu
@pytest.mark.parametrize("world", [1, 8])
def test_gemm_ar_reference_flow(dev, world):
    """bench/gemm_ar_bench.py:429-470: zero C, C_final and ar_done, advance
    the epoch, call (staging_buf is torch.empty there), check C_final
    against the all-reduce of the ranks' matmuls."""
    from oracle.gemm import gemm_ar_ref, rel_fro
    _say(f"ar reference flow world={world}")
    mod = load_module.load("gemm_ar")
    M, K, N = 1024, 256, 512
    A = wl.randn_bf16((M, K), 50, K ** -0.5)
    B = wl.randn_bf16((K, N), 51, K ** -0.5)
    peers = wl.randn_bf16((world - 1, M, N), 52, 0.5)
    C = mod.DistBuffer((M, N), torch.bfloat16, 0, world, True)
    C_final = mod.DistBuffer((M, N), torch.bfloat16, 0, world)
    barrier = mod.DistBuffer((2, 1024, 1024), torch.int32, 0, world, True)
    staging_buf = torch.empty(M // world * N, dtype=torch.bfloat16, device=dev)
    ar_done = torch.zeros(4096, dtype=torch.int32, device=dev)
    ref = gemm_ar_ref(A, B, peers)
    Ad, Bd = A.to(dev), B.to(dev)
    kw = {"peer_partials": peers.to(dev)} if world > 1 else {}
    epoch = 1
    for it in range(3):
        C.data_.zero_(); C_final.data_.zero_(); ar_done.zero_()
        epoch += 1
        mod.set_epoch(epoch)
        mod.gemm_ar_multinode(Ad, Bd, C, barrier, C_final, staging_buf.data_ptr(), mod.get_recv_buf_ptr(),
                              *mod.get_fifo_handles(), mod.get_arrival_flags_ptr(), epoch, 0, 8, 0,
                              ar_done.data_ptr(), arrival_tails_ptr=0, scratch_ints=4096, num_qps=0,
                              num_remote_queues=1, num_allocated_remote_queues=1, cross_node_barrier_ptr=0,
                              use_acquire_poll=False, num_nodes=1, **kw)
        torch.cuda.synchronize()
        assert rel_fro(C_final.data_.float(), ref) < 2e-2, it
        ntiles = (M // 256) * (N // 256)
        assert (ar_done[:ntiles].cpu() != 0).all() and (ar_done[ntiles:].cpu() == 0).all()
        assert (C.data_ == 0).all()


@pytest.mark.gpu
def test_moe_reference_flows(dev):
    from oracle import moe as om
    from oracle.gemm import rel_fro
    _say("moe reference flows")
    cfg = wl.MoeCfg(tokens=512, H=512, I=256, experts=64, topk=8, ep=8, rank=2)
    tokens, ids, gates, w1, w2 = wl.moe_inputs(cfg)
    idx = load_module.build_routing_indices(ids, gates, rank=2, experts=64, ep=8)
    d = {k: torch.from_numpy(np.ascontiguousarray(v)).to(dev) for k, v in idx.items() if isinstance(v, np.ndarray)}
    R_pad, T = idx["R_pad"], cfg.tokens
    post_ref = om.permute_ref(tokens, idx["pull_indices"])
    # dispatch + GEMM1 (bench/dispatch_gemm_bench.py:463-487 checks `outputs`)
    mod = load_module.load("dispatch_gemm")
    pre = mod.DistBuffer((T, cfg.H), torch.bfloat16)
    pre.data_.copy_(tokens.to(dev))
    for write_post in (False, True):
        post = torch.zeros((R_pad, cfg.H), dtype=torch.bfloat16, device=dev)
        out = torch.zeros((R_pad, 2 * cfg.I), dtype=torch.bfloat16, device=dev)
        mod.moe_dispatch_gemm_fused(pre, None, None, post, w1.to(dev), out, d["padded_tokens_per_expert"],
                                    d["pull_indices"], d["local_rb_per_expert"], None, None, 0, 0, 0, 0, 0, 0, 0, 1,
                                    0, T, R_pad, 0, 0, 0, 1, write_post_tokens=write_post)
        torch.cuda.synchronize()
        assert torch.equal(post.cpu(), post_ref if write_post else torch.zeros_like(post_ref))
        assert rel_fro(out.float(), om.grouped_gemm_ref(post_ref, w1, idx["padded_tokens_per_expert"])) < 2e-2
    # full FFN + combine, called twice (tables and session buffers reused)
    mod = load_module.load("dispatch_gemm_glu_combine")
    act = torch.zeros((R_pad, cfg.I), dtype=torch.bfloat16, device=dev)
    ye = torch.zeros((R_pad, cfg.H), dtype=torch.bfloat16, device=dev)
    y_out = mod.DistBuffer((T, cfg.H), torch.float32)
    _, ye_ref = om.ffn_ref(post_ref, w1, w2, idx["padded_tokens_per_expert"], cfg.I)
    y_ref = om.combine_ref(ye_ref, idx["row_weight"], idx["pull_indices"], T)
    for _ in range(2):
        y_out.data_.zero_()
        mod.moe_dispatch_gemm_glu_combine_fused(
            pre, None, None, post, w1.to(dev), w2.to(dev), act, ye, d["row_expert"], d["row_weight"],
            d["padded_tokens_per_expert"], d["pull_indices"], d["local_rb_per_expert"], None, None, y_out, None,
            d["owner_offset"], d["row_to_slot"], d["row_to_owner"], None, None, None, None, 0, 0, 0, 0, 0, 0, 0, 0, 1,
            0, T, R_pad, 0, 0, 0, 1, 1)
        torch.cuda.synchronize()
        assert rel_fro(y_out.data_, y_ref) < 2e-2
