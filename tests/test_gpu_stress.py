"""Randomized arrival orders at the BASELINE sizes: every gated launch must
be bit-equal to the ungated GEMM (AllGather) or to the first launch (reduce
epilogues), in every staging mode, launch after launch on the same flag
arrays with increasing epochs.  Every wait is bounded (spin limit + error
word), so a protocol error fails the test instead of hanging it."""
import pytest
import torch

from mkernel_amd import ops, workloads as wl

pytestmark = pytest.mark.gpu
SPIN = 1 << 24


def _say(msg):
    print(msg, flush=True)


def test_ag_gemm_random_orders_all_modes(dev):
    cfg = wl.AgCfg()
    A, B, _ = wl.ag_inputs(cfg, device=dev)
    A_full = torch.zeros_like(A)
    C = torch.empty((cfg.M, cfg.N), dtype=torch.bfloat16, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    cus = ops.cu_count()
    modes = [-1, -2, 32, -3, -4]
    ref, flags, cnts, ep = {}, {}, {}, {}
    for m in modes:  # ungated on the same number of compute workgroups: the same K-split plan
        ref[m] = torch.empty_like(C)
        ops.ag_gemm(None, A, B, ref[m], None, None, epoch=1, gated=False, num_producers=0, num_cus=cus - max(m, 0))
        flags[m] = torch.zeros(cfg.M // 128, dtype=torch.int32, device=dev)
        cnts[m] = torch.zeros_like(flags[m])
        ep[m] = 0
    for i in range(100):
        m = modes[i % len(modes)]
        ep[m] += 1
        if i % 20 == 0:
            _say(f"ag stress i={i}")
        order = torch.from_numpy(wl.stage_order(cfg.M // 128, 1000 + i)).to(dev)
        A_full.zero_()
        ops.ag_gemm(A, A_full, B, C, flags[m], order, epoch=ep[m], num_producers=m, stage_counters=cnts[m],
                    spin_limit=SPIN, error_word=err)
        assert int(err.item()) == 0, f"i={i} mode={m}: a wait timed out"
        assert torch.equal(A_full, A), f"i={i} mode={m}: staging"
        assert torch.equal(C, ref[m]), f"i={i} mode={m}: gated != ungated"


def test_gemm_rs_random_orders(dev):
    cfg = wl.RsCfg()
    A, B, peers, _ = wl.rs_inputs(cfg, device=dev)
    rows = cfg.M // cfg.world
    work = torch.empty((cfg.M, cfg.N), dtype=torch.bfloat16, device=dev)
    out = torch.empty((rows, cfg.N), dtype=torch.bfloat16, device=dev)
    recv = torch.empty_like(peers)
    nfl = (cfg.world - 1) * rows // 128
    flags = torch.zeros(nfl, dtype=torch.int32, device=dev)
    cnts = torch.zeros_like(flags)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    sent = torch.ones(cfg.M, dtype=torch.bool, device=dev)
    sent[cfg.rank * rows:(cfg.rank + 1) * rows] = False
    first = None
    for i in range(40):
        m = [-1, -3][i % 2]
        if i % 10 == 0:
            _say(f"rs stress i={i}")
        order = torch.from_numpy(wl.stage_order(nfl, 2000 + i)).to(dev)
        ops.gemm_rs(A, B, work, out, peers, recv, cfg.world, cfg.rank, flags, order, epoch=i + 1,
                    num_producers=m, stage_counters=cnts, spin_limit=SPIN, error_word=err)
        assert int(err.item()) == 0, f"i={i} mode={m}: a wait timed out"
        assert torch.equal(recv, peers), f"i={i}: staging"
        if first is None:
            first = (out.clone(), work[sent].clone())
        assert torch.equal(out, first[0]) and torch.equal(work[sent], first[1]), f"i={i} mode={m}"


def test_gemm_ar_two_shot_random_orders(dev):
    M, N, K, world, rank = 8192, 8192, 3584, 8, 3
    A = wl.randn_bf16((M, K), 60, K ** -0.5, dev)
    B = wl.randn_bf16((K, N), 61, K ** -0.5, dev)
    s = M // world
    psrc = wl.randn_bf16((world - 1, s, N), 62, 0.5, dev)
    red = wl.randn_bf16((world - 1, s, N), 63, 1.0, dev)
    recv = torch.empty_like(psrc)
    sends = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    C = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    nb = 2 * (world - 1) * s // 128
    flags = torch.zeros(nb, dtype=torch.int32, device=dev)
    cnts = torch.zeros_like(flags)
    done = torch.zeros((M // 256) * (N // 256), dtype=torch.int32, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    first = None
    for i in range(40):
        m = [-1, -3][i % 2]
        if i % 10 == 0:
            _say(f"ar two-shot stress i={i}")
        order = torch.from_numpy(wl.stage_order(nb, 4000 + i)).to(dev)
        ops.gemm_ar_two_shot(A, B, C, sends, psrc, recv, red, world, rank, flags, order, epoch=i + 1,
                             num_producers=m, stage_counters=cnts, done_flags=done, spin_limit=SPIN, error_word=err)
        assert int(err.item()) == 0, f"i={i} mode={m}: a wait timed out"
        if first is None:
            first = C.clone()
        assert torch.equal(C, first), f"i={i} mode={m}"
