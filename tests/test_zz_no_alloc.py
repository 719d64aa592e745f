"""mk_ag_gemm_noalloc (the allocation-free variant of mk_ag_gemm, scratch in
a static device array) against mk_ag_gemm through the C-ABI: the same
inputs give the same bits, on two calls in a row (the second smaller, so
stale scratch from the first would show), and sizes past the static scratch
are refused."""
import ctypes as C

import pytest
import torch

from mkernel_amd import capi, ops, workloads as wl
from oracle.gemm import ag_gemm_ref, rel_fro

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _args(src, A_full, B, Cout, flags, order, epoch, producers, counters=None, split=(None, 0)):
    M, K = A_full.shape
    N = B.shape[1]
    p = lambda t: None if t is None else t.data_ptr()
    return capi.AgGemmArgs(p(src), p(A_full), p(B), p(Cout), M, N, K, p(flags), p(order), epoch, 1, producers, 0, 0,
                           None, p(counters), split[0], split[1], None, 0)


def _stream():
    return torch.cuda.current_stream().cuda_stream


@pytest.mark.parametrize("producers", [-1, -2, 4, -3])
def test_noalloc_matches_ag_gemm(dev, producers):
    ws = ops.split_workspace(dev)
    for step, (world, rows, K, N, seed) in enumerate([(8, 1024, 1024, 2304, 0), (4, 1024, 512, 4352, 5)]):
        _say(f"noalloc producers={producers} call {step} M={world * rows} K={K} N={N}")
        cfg = wl.AgCfg(world=world, shard_rows=rows, K=K, N=N)
        A, B, order = wl.ag_inputs(cfg, seed=seed)
        Ad, Bd, od = A.to(dev), B.to(dev), torch.from_numpy(order).to(dev)
        nb = cfg.M // 128
        # existing entry point, caller-provided scratch
        full1 = torch.zeros_like(Ad)
        flags1 = torch.zeros(nb, dtype=torch.int32, device=dev)
        cnt1 = torch.zeros_like(flags1)
        C1 = torch.empty((cfg.M, N), dtype=torch.bfloat16, device=dev)
        capi.call("mk_ag_gemm", _args(Ad, full1, Bd, C1, flags1, od, 3, producers, cnt1,
                                      (ws.data_ptr(), ws.numel())), _stream())
        # no-alloc entry point, static scratch
        full2 = torch.zeros_like(Ad)
        flags2 = torch.zeros(nb, dtype=torch.int32, device=dev)
        C2 = torch.full((cfg.M, N), 5.0, dtype=torch.bfloat16, device=dev)
        capi.call("mk_ag_gemm_noalloc", _args(Ad, full2, Bd, C2, flags2, od, 3, producers), _stream())
        torch.cuda.synchronize()
        assert torch.equal(C1, C2), "no-alloc output differs from mk_ag_gemm"
        assert torch.equal(full2, Ad) and (flags2 == 3).all()
        assert rel_fro(C2.float(), ag_gemm_ref(A, B)) < 2e-2


def _split_parts(tiles, K):
    """Partial tiles the library's K-split plan writes for `tiles` 256x256
    tiles on every CU (the rule of plan_split)."""
    cus = ops.cu_count()
    R = tiles % cus
    if R == 0:
        return 0
    s = min(4, cus // R, (K // 32) // 4)
    return R * (s - 1) if s >= 2 else 0


def test_noalloc_tail_split_beyond_static_scratch_runs_unsplit(dev):
    """A tail round whose K-split needs more partial tiles than the static
    scratch holds (128) runs unsplit: bit-equal to mk_ag_gemm without a
    K-split workspace.  A second call with a split that fits follows."""
    for world, rows, K, N in [(8, 512, 512, 5120), (8, 1024, 1024, 2304)]:
        M = world * rows
        parts = _split_parts((M // 256) * (N // 256), K)
        _say(f"noalloc split parts={parts} M={M} K={K} N={N}")
        cfg = wl.AgCfg(world=world, shard_rows=rows, K=K, N=N)
        A, B, order = wl.ag_inputs(cfg, seed=9)
        Ad, Bd, od = A.to(dev), B.to(dev), torch.from_numpy(order).to(dev)
        nb = M // 128
        full1, full2 = torch.zeros_like(Ad), torch.zeros_like(Ad)
        flags1 = torch.zeros(nb, dtype=torch.int32, device=dev)
        flags2 = torch.zeros_like(flags1)
        cnt1 = torch.zeros_like(flags1)
        C1 = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        C2 = torch.full_like(C1, 3.0)
        ws = ops.split_workspace(dev)
        split = (None, 0) if parts > 128 else (ws.data_ptr(), ws.numel())
        capi.call("mk_ag_gemm", _args(Ad, full1, Bd, C1, flags1, od, 2, -1, cnt1, split), _stream())
        capi.call("mk_ag_gemm_noalloc", _args(Ad, full2, Bd, C2, flags2, od, 2, -1), _stream())
        torch.cuda.synchronize()
        assert torch.equal(C1, C2)
        assert torch.equal(full2, Ad)


def test_noalloc_present_blocks(dev):
    """n_present through the no-alloc entry point: the own shard's blocks
    are published without a copy (junk in their source rows never reaches
    A_full or C), bit-equal to mk_ag_gemm."""
    world, rows, K, N, rank = 8, 512, 512, 1024, 2
    cfg = wl.AgCfg(world=world, shard_rows=rows, K=K, N=N)
    A, B, order = wl.ag_inputs(cfg, seed=4)
    per = rows // 128
    own = list(range(rank * per, (rank + 1) * per))
    od = torch.tensor(own + [int(b) for b in order if int(b) not in own], dtype=torch.int32, device=dev)
    src = A.clone()
    src[rank * rows:(rank + 1) * rows] = float("nan")
    outs = []
    for entry in ("mk_ag_gemm", "mk_ag_gemm_noalloc"):
        _say(f"noalloc n_present via {entry}")
        full = torch.zeros_like(A)
        full[rank * rows:(rank + 1) * rows] = A[rank * rows:(rank + 1) * rows]
        full = full.to(dev)
        flags = torch.zeros(cfg.M // 128, dtype=torch.int32, device=dev)
        Cout = torch.empty((cfg.M, N), dtype=torch.bfloat16, device=dev)
        if entry == "mk_ag_gemm":
            ws = ops.split_workspace(dev)
            args = _args(src.to(dev), full, B.to(dev), Cout, flags, od, 6, -1, torch.zeros_like(flags),
                         (ws.data_ptr(), ws.numel()))
        else:
            args = _args(src.to(dev), full, B.to(dev), Cout, flags, od, 6, -1)
        args.n_present = per
        capi.call(entry, args, _stream())
        torch.cuda.synchronize()
        assert torch.equal(full.cpu(), A) and (flags == 6).all()
        outs.append(Cout.cpu())
    assert torch.equal(outs[0], outs[1])


def test_noalloc_graph_replays(dev):
    """The no-alloc call recorded in a HIP graph after mk_epoch_advance:
    every replay (new shard contents written between replays) clears its
    scratch with a kernel, stages under a new epoch and gives the ungated
    GEMM's bits."""
    cfg = wl.AgCfg(world=8, shard_rows=256, K=512, N=512)
    A, B, order = wl.ag_inputs(cfg, seed=2)
    shards = A.to(dev)
    Bd, od = B.to(dev), torch.from_numpy(order).to(dev)
    A_full = torch.zeros_like(shards)
    Cout = torch.empty((cfg.M, cfg.N), dtype=torch.bfloat16, device=dev)
    flags = torch.zeros(cfg.M // 128, dtype=torch.int32, device=dev)
    word = torch.zeros(1, dtype=torch.int32, device=dev)
    args = _args(shards, A_full, Bd, Cout, flags, od, 0, -1)
    args.epoch_ptr = word.data_ptr()

    def step():
        ops.epoch_advance(word)
        capi.call("mk_ag_gemm_noalloc", args, _stream())

    _say("noalloc graph capture")
    step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    gen = torch.Generator().manual_seed(3)
    for rep in range(3):
        _say(f"noalloc graph replay {rep}")
        new = (torch.randn(cfg.M, cfg.K, generator=gen) / cfg.K ** 0.5).to(torch.bfloat16)
        shards.copy_(new.to(dev))
        g.replay()
        torch.cuda.synchronize()
        assert int(word.item()) == 2 + rep and (flags.cpu() == 2 + rep).all()
        assert torch.equal(A_full.cpu(), new)
        ref = torch.empty_like(Cout)
        ops.ag_gemm(None, A_full, Bd, ref, None, None, epoch=1, gated=False, num_producers=0)
        torch.cuda.synchronize()
        assert torch.equal(Cout, ref)


def test_noalloc_refuses_out_of_range(dev):
    _say("noalloc refusals")
    L = capi.lib()
    assert L.mk_ag_gemm_noalloc_scratch_bytes() > 0
    t = torch.zeros(256, dtype=torch.bfloat16, device=dev)
    big = capi.AgGemmArgs(t.data_ptr(), t.data_ptr(), t.data_ptr(), t.data_ptr(), 128 * 16385, 256, 256,
                          t.data_ptr(), t.data_ptr(), 1, 1, -1, 0, 0, None, None, None, 0, None, 0)
    with pytest.raises(capi.MkError, match="static scratch"):
        capi.call("mk_ag_gemm_noalloc", big, _stream())
    ws = capi.AgGemmArgs(t.data_ptr(), t.data_ptr(), t.data_ptr(), t.data_ptr(), 256, 256, 256,
                         t.data_ptr(), t.data_ptr(), 1, 1, -1, 0, 0, None, t.data_ptr(), None, 0, None, 0)
    with pytest.raises(capi.MkError, match="NULL"):
        capi.call("mk_ag_gemm_noalloc", ws, _stream())
    torch.cuda.synchronize()
