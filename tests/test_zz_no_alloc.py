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


@pytest.mark.parametrize("producers", [-1, -2, 4])
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
