"""GPU parity of the GEMM core, the flag-gated AllGather consumer and the
reduce-scatter epilogue against the CPU oracle (all through the C-ABI)."""
import ctypes as C

import numpy as np
import pytest
import torch

from mkernel_amd import ops, workloads as wl
from mkernel_amd.capi import MkError
from oracle.gemm import ag_gemm_ref, gemm_ref, gemm_rs_ref, rel_fro

pytestmark = pytest.mark.gpu
TOL = 2e-2  # rel-Frobenius bound from BASELINE north_star


def _say(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("waves", [4, 8])
@pytest.mark.parametrize("M,N,K,tile", [(128, 256, 64, 128), (256, 256, 128, 256), (512, 512, 512, 0),
                                        (384, 768, 1024, 128), (1024, 1280, 320, 256), (256, 512, 32, 256),
                                        (128, 256, 96, 128)])
def test_gemm_vs_oracle(dev, M, N, K, tile, waves):
    _say(f"gemm M={M} N={N} K={K} tile={tile} waves={waves}")
    A = wl.randn_bf16((M, K), 10, K ** -0.5)
    B = wl.randn_bf16((K, N), 11, K ** -0.5)
    C = ops.gemm(A.to(dev), B.to(dev), tile_m=tile, waves=waves)
    torch.cuda.synchronize()
    assert rel_fro(C.float(), gemm_ref(A, B)) < TOL
    # each output is the fp32 dot product rounded once to bf16
    ref = gemm_ref(A, B)
    assert torch.allclose(C.cpu().float(), ref, rtol=2 ** -7, atol=1e-5)


@pytest.mark.parametrize("waves", [4, 8])
@pytest.mark.parametrize("tile", [128, 256])
def test_gemm_identity_is_exact(dev, tile, waves):
    """I @ B == B and A @ I == A bit-exactly (pins the operand/accumulator layout)."""
    _say(f"gemm identity tile={tile} waves={waves}")
    n = 512
    I = torch.eye(n, dtype=torch.bfloat16)
    X = wl.randn_bf16((n, n), 12)
    assert torch.equal(ops.gemm(I.to(dev), X.to(dev), tile_m=tile, waves=waves).cpu(), X)
    assert torch.equal(ops.gemm(X.to(dev), I.to(dev), tile_m=tile, waves=waves).cpu(), X)


def test_gemm_permutation_exact(dev):
    """A permutation matrix on the left permutes rows of B exactly."""
    n = 256
    perm = torch.randperm(n, generator=torch.Generator().manual_seed(3))
    P = torch.zeros(n, n, dtype=torch.bfloat16)
    P[torch.arange(n), perm] = 1
    X = wl.randn_bf16((n, 512), 13)
    assert torch.equal(ops.gemm(P.to(dev), X.to(dev)).cpu(), X[perm])


@pytest.mark.parametrize("M,N,K,tile,cus", [(1024, 2560, 1024, 256, 0), (768, 1024, 2048, 128, 0),
                                             (1024, 2560, 512, 256, 96), (2048, 2048, 1024, 256, 200)])
def test_gemm_split_tail(dev, M, N, K, tile, cus):
    """Tail round split along K through the workspace: matches the oracle and
    the unsplit GEMM, twice in a row on one workspace (flags left zeroed)."""
    _say(f"gemm split M={M} N={N} K={K} tile={tile} cus={cus}")
    A = wl.randn_bf16((M, K), 20, K ** -0.5).to(dev)
    B = wl.randn_bf16((K, N), 21, K ** -0.5).to(dev)
    ws = torch.zeros(int(ops.capi.lib().mk_query_workspace_bytes(0, M, N, K)), dtype=torch.uint8, device=dev)
    plain = ops.gemm(A, B, tile_m=tile, num_cus=cus, split_ws=False)
    ref = gemm_ref(A.cpu(), B.cpu())
    for _ in range(2):
        C = ops.gemm(A, B, tile_m=tile, num_cus=cus, split_ws=ws)
        torch.cuda.synchronize()
        assert rel_fro(C.float(), ref) < TOL
        assert torch.allclose(C.cpu().float(), ref, rtol=2 ** -7, atol=1e-5)
        # fp32 partial sums differ from the unsplit order by fp32 rounding only
        assert torch.allclose(C.float(), plain.float(), rtol=2 ** -7, atol=1e-5)
    assert int(ws[:4096].view(torch.int32).abs().sum()) == 0, "split flags not left zeroed"


@pytest.mark.parametrize("M,N,K,cus", [(8192, 3584, 256, 0),    # 448 tiles: one round + 192 spread over the XCDs
                                       (4096, 3584, 512, 0),    # 224 tiles: one partial round
                                       (4096, 3584, 256, 128),  # 224 on 128: one round + 96
                                       (4096, 3584, 256, 130)])  # grid not a multiple of 8: consumer order
def test_gemm_partial_round_every_tile(dev, M, N, K, cus):
    """A partial last round of whole tiles (too many tiles to K-split) is
    dealt to consumers spread over the XCDs: every tile is written once and
    matches the oracle, and the result is bit-equal across grids."""
    _say(f"gemm partial round M={M} N={N} K={K} cus={cus}")
    A = wl.randn_bf16((M, K), 23, K ** -0.5)
    B = wl.randn_bf16((K, N), 24, K ** -0.5)
    C = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
    ops.gemm(A.to(dev), B.to(dev), C, num_cus=cus, tile_m=256)
    torch.cuda.synchronize()
    ref = gemm_ref(A, B)
    assert not torch.isnan(C).any(), "a tile of the partial round was not written"
    assert torch.allclose(C.cpu().float(), ref, rtol=2 ** -7, atol=1e-5)
    # 256-row tiles, no K-split on these shapes: every element is one fp32
    # dot product in K order, so any grid gives the same bits
    C8 = ops.gemm(A.to(dev), B.to(dev), num_cus=8, tile_m=256)
    assert torch.equal(C, C8)


def test_gemm_random_shapes_and_grids(dev):
    """Seeded random shapes, grid sizes and tile heights: whatever mix of
    whole rounds, spread partial rounds and K-split tails the planner picks,
    every output matches the oracle (one fp32 dot product per element up to
    the split's fp32 rounding) and no tile is left unwritten."""
    rng = np.random.default_rng(2024)
    cus = ops.cu_count()
    for case in range(16):
        M = int(rng.integers(1, 17)) * 256
        N = int(rng.integers(1, 13)) * 256
        K = int(rng.integers(1, 33)) * 32
        grid = int(rng.choice([0, 0, 8, 24, 64, 96, 130, 200, cus]))
        tile = int(rng.choice([0, 128, 256]))
        _say(f"gemm random case={case} M={M} N={N} K={K} grid={grid} tile={tile}")
        A = wl.randn_bf16((M, K), 100 + case, K ** -0.5)
        B = wl.randn_bf16((K, N), 200 + case, K ** -0.5)
        C = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
        ops.gemm(A.to(dev), B.to(dev), C, num_cus=grid, tile_m=tile)
        torch.cuda.synchronize()
        assert not torch.isnan(C).any(), f"case {case}: unwritten tiles"
        ref = gemm_ref(A, B)
        assert rel_fro(C.float(), ref) < TOL, f"case {case}"
        assert torch.allclose(C.cpu().float(), ref, rtol=2 ** -6, atol=1e-4), f"case {case}"


def test_gemm_split_identity_exact(dev):
    """With a 4-way K split, I @ X is still exact (partials are exact sums)."""
    n = 1024
    I = torch.eye(n, dtype=torch.bfloat16, device=dev)
    X = wl.randn_bf16((n, n), 22).to(dev)
    assert torch.equal(ops.gemm(I, X, tile_m=256).cpu(), X.cpu())
    assert torch.equal(ops.gemm(X, I, tile_m=128).cpu(), X.cpu())


def test_gemm_bad_shape_raises(dev):
    A = torch.zeros((100, 64), dtype=torch.bfloat16, device=dev)
    B = torch.zeros((64, 256), dtype=torch.bfloat16, device=dev)
    with pytest.raises(MkError):
        ops.gemm(A, B)


def test_gemm_config1_slice(dev):
    """Config 1 at full size (4096^3): a 256-row slice against the oracle."""
    _say("gemm config1 4096^3")
    A, B = wl.gemm_inputs(wl.GemmCfg(), device="cpu")
    C = ops.gemm(A.to(dev), B.to(dev))
    torch.cuda.synchronize()
    rows = slice(1024, 1280)
    assert rel_fro(C[rows].float(), gemm_ref(A[rows], B)) < TOL
    assert torch.isfinite(C.float()).all()


def _ag_case(dev, world=8, shard=256, K=512, N=512, seed=0):
    cfg = wl.AgCfg(world=world, shard_rows=shard, K=K, N=N)
    A, B, order = wl.ag_inputs(cfg, seed=seed)
    return cfg, A, B, torch.from_numpy(order)


@pytest.mark.parametrize("producers", [-1, -2, 1, 4, 16, -3, -4, -6])
def test_ag_gemm_producer_gated(dev, producers):
    _say(f"ag_gemm producers={producers}")
    cfg, A, B, order = _ag_case(dev)
    Ad, Bd = A.to(dev), B.to(dev)
    A_full = torch.zeros_like(Ad)
    flags = torch.zeros(cfg.M // 128, dtype=torch.int32, device=dev)
    counters = torch.zeros(cfg.M // 128, dtype=torch.int32, device=dev)
    C = torch.empty((cfg.M, cfg.N), dtype=torch.bfloat16, device=dev)
    ops.ag_gemm(Ad, A_full, Bd, C, flags, order.to(dev), epoch=1, num_producers=producers, stage_counters=counters)
    torch.cuda.synchronize()
    assert torch.equal(A_full.cpu(), A)  # staging is a bit-exact copy
    assert (flags.cpu() == 1).all()
    ref = ag_gemm_ref(A, B)
    assert rel_fro(C.float(), ref) < TOL
    # flag order must not change the result (bit-equal to the ungated GEMM)
    C2 = torch.empty_like(C)
    ops.ag_gemm(None, A_full, Bd, C2, None, None, epoch=1, gated=False, num_producers=0)
    torch.cuda.synchronize()
    assert torch.equal(C.cpu(), C2.cpu())
    if producers <= -3:
        # the co-resident staging leaves its claim words (the last 64 bytes of
        # the K-split flag area) zeroed for the next launch
        ws = ops.split_workspace(dev)
        assert int(ws[4096 - 64:4096].cpu().count_nonzero()) == 0


def test_ag_gemm_random_shapes_and_grids(dev):
    """Seeded random AllGather shapes, grids and producer modes: the staged
    A_full is a bit-exact copy, every flag is published, and the gated
    result is bit-equal to the ungated GEMM on the same grid (same K-split
    plan), whatever rounds, spread partial rounds and tails the plan has."""
    rng = np.random.default_rng(77)
    for case in range(10):
        world = int(rng.choice([2, 4, 8]))
        shard = int(rng.integers(1, 9)) * 256
        N = int(rng.integers(1, 15)) * 256
        K = int(rng.integers(1, 17)) * 64
        grid = int(rng.choice([0, 0, 16, 64, 128, 200]))
        prod = int(rng.choice([-1, -2, 4]))
        cfg = wl.AgCfg(world=world, shard_rows=shard, K=K, N=N)
        _say(f"ag_gemm random case={case} world={world} M={cfg.M} N={N} K={K} grid={grid} prod={prod}")
        A, B, order = wl.ag_inputs(cfg, seed=300 + case)
        Ad, Bd = A.to(dev), B.to(dev)
        A_full = torch.zeros_like(Ad)
        flags = torch.zeros(cfg.M // 128, dtype=torch.int32, device=dev)
        counters = torch.zeros_like(flags)
        C = torch.empty((cfg.M, N), dtype=torch.bfloat16, device=dev)
        ops.ag_gemm(Ad, A_full, Bd, C, flags, torch.from_numpy(order).to(dev), epoch=3, num_producers=prod,
                    num_cus=grid, stage_counters=counters)
        # the same number of compute workgroups (dedicated producers take
        # grid slots), hence the same K-split plan
        compute = (grid or ops.cu_count()) - max(prod, 0)
        C2 = torch.empty_like(C)
        ops.ag_gemm(None, A_full, Bd, C2, None, None, epoch=1, gated=False, num_producers=0, num_cus=compute)
        torch.cuda.synchronize()
        assert torch.equal(A_full.cpu(), A), f"case {case}: staging"
        assert (flags.cpu() == 3).all(), f"case {case}: flags"
        assert torch.equal(C.cpu(), C2.cpu()), f"case {case}: gated != ungated"
        assert rel_fro(C.float(), ag_gemm_ref(A, B)) < TOL, f"case {case}"


def test_ag_gemm_epochs_and_orders(dev):
    """Several calls with increasing (and skipped) epochs, different stage
    orders and both staging modes, no flag or counter reset in between:
    every result is bit-identical."""
    cfg, A, B, _ = _ag_case(dev)
    Ad, Bd = A.to(dev), B.to(dev)
    flags = torch.zeros(cfg.M // 128, dtype=torch.int32, device=dev)
    counters = torch.zeros(cfg.M // 128, dtype=torch.int32, device=dev)
    outs = []
    for epoch, seed, prod in [(1, 5, -1), (2, 6, 8), (5, 7, -1), (6, 8, -1), (7, 9, -3), (9, 10, -3), (11, 11, -4),
                              (12, 12, -1)]:
        _say(f"ag_gemm epoch={epoch} producers={prod}")
        A_full = torch.zeros_like(Ad)
        order = torch.from_numpy(wl.stage_order(cfg.M // 128, seed)).to(dev)
        C = torch.empty((cfg.M, cfg.N), dtype=torch.bfloat16, device=dev)
        ops.ag_gemm(Ad, A_full, Bd, C, flags, order, epoch=epoch, num_producers=prod, stage_counters=counters)
        torch.cuda.synchronize()
        assert torch.equal(A_full.cpu(), A)
        assert (flags.cpu() == epoch).all()
        outs.append(C.cpu())
    assert all(torch.equal(outs[0], o) for o in outs[1:])


@pytest.mark.parametrize("num_cus,K,prod", [(4, 512, -1), (8, 1024, -1), (8, 1024, -2), (16, 512, -1), (3, 2048, -1),
                                            (0, 512, -1), (3, 2048, -3), (8, 1024, -3), (16, 512, -6)])
def test_ag_gemm_cooperative_staging_capped_grid(dev, num_cus, K, prod):
    """Cooperative staging with a capped grid (every workgroup copies many
    pieces and computes several rounds of tiles): staged bytes and flags
    exact, result bit-equal to the ungated GEMM, over several epochs.  With
    3 workgroups the 16 tiles leave one tail tile, split 3 ways along K while
    whole tiles follow the arrival order (a regression case: a whole tile at
    a permuted position past the split boundary once waited on the split
    flags).  Waits are bounded so a protocol error reports instead of
    hanging.  num_cus 8 and 16 (multiples of the 8 XCDs) run the schedule in
    which the two halves of the grid take turns copying ahead (-1); -2 the
    even share; -3 and -6 the co-resident staging kernel (1 and 4 staging
    waves per workgroup) sharing the claimed pieces with the compute
    workgroups."""
    _say(f"ag_gemm cooperative num_cus={num_cus} K={K} producers={prod}")
    cfg, A, B, order = _ag_case(dev, K=K)
    Ad, Bd = A.to(dev), B.to(dev)
    flags = torch.zeros(cfg.M // 128, dtype=torch.int32, device=dev)
    counters = torch.zeros_like(flags)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    C_ref = torch.empty((cfg.M, cfg.N), dtype=torch.bfloat16, device=dev)
    ops.ag_gemm(None, Ad, Bd, C_ref, None, None, epoch=1, gated=False, num_producers=0, num_cus=num_cus,
                spin_limit=4_000_000, error_word=err)
    for epoch in (1, 2, 4):
        A_full = torch.zeros_like(Ad)
        C = torch.empty_like(C_ref)
        ops.ag_gemm(Ad, A_full, Bd, C, flags, order.to(dev), epoch=epoch, num_producers=prod, num_cus=num_cus,
                    stage_counters=counters, spin_limit=4_000_000, error_word=err)
        torch.cuda.synchronize()
        assert int(err.item()) == 0, "a bounded wait timed out"
        assert torch.equal(A_full.cpu(), A)
        assert (flags.cpu() == epoch).all()
        assert torch.equal(C.cpu(), C_ref.cpu())
    assert rel_fro(C_ref.float(), ag_gemm_ref(A, B)) < TOL


def test_ag_gemm_preset_flags(dev):
    """Flags published by someone else (no producer role in the launch)."""
    cfg, A, B, order = _ag_case(dev)
    flags = torch.full((cfg.M // 128,), 7, dtype=torch.int32, device=dev)
    C = torch.empty((cfg.M, cfg.N), dtype=torch.bfloat16, device=dev)
    ops.ag_gemm(None, A.to(dev), B.to(dev), C, flags, order.to(dev), epoch=7, num_producers=0)
    torch.cuda.synchronize()
    assert rel_fro(C.float(), ag_gemm_ref(A, B)) < TOL


def test_ag_gemm_bounded_wait_reports_timeout(dev):
    """A flag nobody publishes: the bounded wait gives up and sets the error
    word instead of hanging (every wave still exits)."""
    cfg, A, B, order = _ag_case(dev)
    flags = torch.zeros(cfg.M // 128, dtype=torch.int32, device=dev)
    flags[: cfg.M // 256] = 3  # half the tiles published, the rest never
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    C = torch.empty((cfg.M, cfg.N), dtype=torch.bfloat16, device=dev)
    ops.ag_gemm(None, A.to(dev), B.to(dev), C, flags, None, epoch=3, num_producers=0, spin_limit=64,
                error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) & 1
    # the published half is still computed correctly
    half = cfg.M // 2
    assert rel_fro(C[:half].float(), gemm_ref(A[:half], B)) < TOL


@pytest.mark.parametrize("rank,producers,num_cus,K", [(0, 4, 0, 256), (3, 8, 0, 256), (7, 0, 0, 256), (5, -1, 0, 256),
                                                     (2, -1, 4, 1024), (6, -1, 3, 256), (1, -1, 5, 2048),
                                                     (4, -3, 0, 256), (3, -4, 8, 512)])
def test_gemm_rs_vs_oracle(dev, rank, producers, num_cus, K):
    _say(f"gemm_rs rank={rank} producers={producers} num_cus={num_cus} K={K}")
    cfg = wl.RsCfg(world=8, rank=rank, M=2048, K=K, N=512)
    A, B, peers, order = wl.rs_inputs(cfg)
    rows = cfg.M // cfg.world
    Ad, Bd = A.to(dev), B.to(dev)
    work = torch.zeros((cfg.M, cfg.N), dtype=torch.bfloat16, device=dev)
    out = torch.zeros((rows, cfg.N), dtype=torch.bfloat16, device=dev)
    nfl = (cfg.world - 1) * rows // 128
    if producers:
        recv = torch.zeros_like(peers, device=dev)
        flags = torch.zeros(nfl, dtype=torch.int32, device=dev)
    else:
        recv = peers.to(dev)
        flags = torch.full((nfl,), 9, dtype=torch.int32, device=dev)
    counters = torch.zeros(nfl, dtype=torch.int32, device=dev)
    ops.gemm_rs(Ad, Bd, work, out, peers.to(dev), recv, cfg.world, rank, flags, torch.from_numpy(order).to(dev),
                epoch=9, num_producers=producers, stage_counters=counters, num_cus=num_cus)
    torch.cuda.synchronize()
    P, owned = gemm_rs_ref(A, B, peers, rank, cfg.world)
    assert rel_fro(out.float(), owned) < TOL
    mask = torch.ones(cfg.M, dtype=torch.bool)
    mask[rank * rows:(rank + 1) * rows] = False
    assert rel_fro(work.cpu()[mask].float(), P[mask]) < TOL
    assert (work.cpu()[~mask] == 0).all()  # owned rows are not sent
    if producers:
        assert torch.equal(recv.cpu(), peers)


def test_gemm_rs_random_shapes_and_grids(dev):
    """Seeded random reduce-scatter shapes, ranks, grids and staging modes:
    the owned slice matches the oracle (fp32 fold, one rounding), the
    non-owned rows are the local partials, the owned rows are not sent, and
    staged partials are bit-exact copies."""
    rng = np.random.default_rng(91)
    for case in range(8):
        world = int(rng.choice([2, 4, 8]))
        rank = int(rng.integers(0, world))
        M = world * int(rng.integers(1, 5)) * 256
        N = int(rng.integers(1, 9)) * 256
        K = int(rng.integers(1, 17)) * 64
        grid = int(rng.choice([0, 0, 16, 64, 136]))
        prod = int(rng.choice([-1, 0, 4]))
        _say(f"gemm_rs random case={case} world={world} rank={rank} M={M} N={N} K={K} grid={grid} prod={prod}")
        cfg = wl.RsCfg(world=world, rank=rank, M=M, K=K, N=N)
        A, B, peers, order = wl.rs_inputs(cfg, seed=400 + case)
        rows = M // world
        nfl = (world - 1) * rows // 128
        work = torch.zeros((M, N), dtype=torch.bfloat16, device=dev)
        out = torch.zeros((rows, N), dtype=torch.bfloat16, device=dev)
        if prod:
            recv = torch.zeros_like(peers, device=dev)
            flags = torch.zeros(nfl, dtype=torch.int32, device=dev)
        else:
            recv = peers.to(dev)
            flags = torch.full((nfl,), 5, dtype=torch.int32, device=dev)
        counters = torch.zeros(nfl, dtype=torch.int32, device=dev)
        ops.gemm_rs(A.to(dev), B.to(dev), work, out, peers.to(dev), recv, world, rank, flags,
                    torch.from_numpy(order).to(dev), epoch=5, num_producers=prod, stage_counters=counters,
                    num_cus=grid)
        torch.cuda.synchronize()
        P, owned = gemm_rs_ref(A, B, peers, rank, world)
        assert rel_fro(out.float(), owned) < TOL, f"case {case}: owned slice"
        mask = torch.ones(M, dtype=torch.bool)
        mask[rank * rows:(rank + 1) * rows] = False
        assert rel_fro(work.cpu()[mask].float(), P[mask]) < TOL, f"case {case}: sends"
        assert (work.cpu()[~mask] == 0).all(), f"case {case}: owned rows sent"
        if prod:
            assert torch.equal(recv.cpu(), peers), f"case {case}: staging"


@pytest.mark.parametrize("world,rank,M,num_cus", [(8, 3, 4096, 0), (4, 0, 2048, 8), (8, 7, 4096, 16), (2, 1, 1024, 0)])
def test_gemm_rs_spread_schedule_orders(dev, world, rank, M, num_cus):
    """Owned row tiles run one per round in the arrival order of their peer
    blocks: with the partials staged inside the launch in a row-block-major
    order, in a random order, and pre-staged with published flags, the owned
    slice and the sends are bit-identical (each owned element is the same
    fp32 sum in rank order whatever round folds it), and match the oracle."""
    _say(f"gemm_rs spread world={world} rank={rank} M={M} num_cus={num_cus}")
    cfg = wl.RsCfg(world=world, rank=rank, M=M, K=256, N=512)
    A, B, peers, order = wl.rs_inputs(cfg)
    rows = cfg.M // cfg.world
    rbs = rows // 128
    Ad, Bd, pd = A.to(dev), B.to(dev), peers.to(dev)
    nfl = (world - 1) * rbs
    row_major = torch.tensor([q * rbs + rb for rb in range(rbs) for q in range(world - 1)], dtype=torch.int32)
    results = []
    for mode, od in (("rows", row_major), ("random", torch.from_numpy(order)), ("prestaged", None)):
        work = torch.zeros((cfg.M, cfg.N), dtype=torch.bfloat16, device=dev)
        out = torch.zeros((rows, cfg.N), dtype=torch.bfloat16, device=dev)
        counters = torch.zeros(nfl, dtype=torch.int32, device=dev)
        if mode == "prestaged":
            ops.gemm_rs(Ad, Bd, work, out, None, pd.clone(), world, rank, torch.full((nfl,), 5, dtype=torch.int32,
                        device=dev), torch.from_numpy(order).to(dev), epoch=5, num_producers=0, num_cus=num_cus)
        else:
            recv = torch.zeros_like(pd)
            ops.gemm_rs(Ad, Bd, work, out, pd, recv, world, rank, torch.zeros(nfl, dtype=torch.int32, device=dev),
                        od.to(dev), epoch=5, num_producers=-1, stage_counters=counters, num_cus=num_cus)
            torch.cuda.synchronize()
            assert torch.equal(recv.cpu(), peers)
        torch.cuda.synchronize()
        results.append((work.cpu(), out.cpu()))
    for w, o in results[1:]:
        assert torch.equal(w, results[0][0]) and torch.equal(o, results[0][1])
    _, owned = gemm_rs_ref(A, B, peers, rank, world)
    assert rel_fro(results[0][1].float(), owned) < TOL


def test_gemm_rs_equal_partials_known_answer(dev):
    """All 8 partials equal => output is exactly 8x the partial.  Integer
    operands in {-1, 0, 1} make every partial an exact small integer."""
    M, K, N, world, rank = 2048, 128, 256, 8, 2
    g = torch.Generator().manual_seed(4)
    A = torch.randint(-1, 2, (M, K), generator=g).to(torch.bfloat16)
    B = torch.randint(-1, 2, (K, N), generator=g).to(torch.bfloat16)
    rows = M // world
    P = (A.float() @ B.float())
    own = P[rank * rows:(rank + 1) * rows]
    peers = own.to(torch.bfloat16).unsqueeze(0).repeat(world - 1, 1, 1).contiguous()
    work = torch.zeros((M, N), dtype=torch.bfloat16, device=dev)
    out = torch.zeros((rows, N), dtype=torch.bfloat16, device=dev)
    ops.gemm_rs(A.to(dev), B.to(dev), work, out, None, peers.to(dev), world, rank, None, None, epoch=1, gated=False,
                num_producers=0)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), (own * world).to(torch.bfloat16))


@pytest.mark.parametrize("producers,num_cus,M,N,K", [(-1, 0, 1024, 512, 256), (4, 0, 1024, 512, 256),
                                                     (-1, 6, 2048, 768, 512), (0, 0, 512, 512, 128),
                                                     (-3, 0, 1024, 512, 256), (-6, 16, 2048, 768, 512)])
def test_gemm_ar_vs_oracle(dev, producers, num_cus, M, N, K):
    """GEMM + all-reduce: C_final = A@B + sum of 7 staged peer partials over
    all rows; staged bytes exact, every output tile published with the
    epoch; arrival order of the peer blocks does not change a bit."""
    _say(f"gemm_ar producers={producers} num_cus={num_cus} M={M} N={N} K={K}")
    world = 8
    A = wl.randn_bf16((M, K), 40, K ** -0.5)
    B = wl.randn_bf16((K, N), 41, K ** -0.5)
    peers = wl.randn_bf16((world - 1, M, N), 42, 0.5)
    nflags = (world - 1) * M // 128
    ntiles = (M // 256) * (N // 256)
    ref = ag_ref = None
    outs = []
    for epoch, seed in [(3, 1), (4, 2)]:
        order = torch.from_numpy(wl.stage_order(nflags, seed)).to(dev)
        recv = torch.zeros((world - 1, M, N), dtype=torch.bfloat16, device=dev)
        flags = torch.zeros(nflags, dtype=torch.int32, device=dev)
        counters = torch.zeros_like(flags)
        done = torch.zeros(ntiles, dtype=torch.int32, device=dev)
        err = torch.zeros(1, dtype=torch.int32, device=dev)
        C = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        if producers == 0:  # partials already in place, flags published by someone else
            recv.copy_(peers.to(dev))
            flags.fill_(epoch)
        ops.gemm_ar(A.to(dev), B.to(dev), C, peers.to(dev) if producers != 0 else None, recv, world, flags, order,
                    epoch=epoch, num_producers=producers, num_cus=num_cus, stage_counters=counters, done_flags=done,
                    spin_limit=4_000_000, error_word=err)
        torch.cuda.synchronize()
        assert int(err.item()) == 0, "a bounded wait timed out"
        assert torch.equal(recv.cpu(), peers), "staged partials differ"
        assert (done.cpu() == epoch).all(), "an output tile was not published"
        outs.append(C.cpu())
    from oracle.gemm import gemm_ar_ref
    ref = gemm_ar_ref(A, B, peers)
    assert rel_fro(outs[0].float(), ref) < TOL
    assert torch.allclose(outs[0].float(), ref, rtol=2 ** -7, atol=1e-2)
    assert torch.equal(outs[0], outs[1]), "result depends on the stage order"


@pytest.mark.parametrize("world,rank,producers,num_cus", [(8, 3, -1, 0), (8, 0, 4, 0), (4, 2, -3, 0), (8, 7, 0, 0),
                                                        (2, 1, -1, 8), (8, 5, -1, 3)])
def test_gemm_ar_two_shot_vs_oracle(dev, world, rank, producers, num_cus):
    """Two-shot all-reduce at one rank's share: the rank's own slice is
    A@B + the world-1 peer partials of that slice (fp32 adds, oracle
    tolerance), every other slice is the peers' reduced rows copied in bit
    for bit, the sends hold this rank's partial rows of the other slices,
    every staged block's flag and every own tile's done flag carry the
    epoch.  producers 0: everything staged before the launch."""
    _say(f"gemm_ar two-shot world={world} rank={rank} producers={producers} num_cus={num_cus}")
    M, N, K = 512 * world // 2 if world > 2 else 1024, 512, 256
    s = M // world
    A = wl.randn_bf16((M, K), 70, K ** -0.5)
    B = wl.randn_bf16((K, N), 71, K ** -0.5)
    P = wl.randn_bf16((world - 1, M, N), 72, 0.5)  # the peers' full partials, rank order without `rank`
    own = gemm_ref(A, B)
    others = [j for j in range(world) if j != rank]
    peer_src = P[:, rank * s:(rank + 1) * s].contiguous()
    reduced = torch.stack([(own[j * s:(j + 1) * s] + P[:, j * s:(j + 1) * s].float().sum(0)).to(torch.bfloat16)
                           for j in others])
    ref_own = own[rank * s:(rank + 1) * s].clone()
    for q in range(world - 1):
        ref_own += peer_src[q].float()
    nb = 2 * (world - 1) * s // 128
    C_final = torch.zeros((M, N), dtype=torch.bfloat16, device=dev)
    sends = torch.zeros((M, N), dtype=torch.bfloat16, device=dev)
    done = torch.zeros((M // 256) * (N // 256), dtype=torch.int32, device=dev)
    counters = torch.zeros(nb, dtype=torch.int32, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    order = torch.from_numpy(wl.stage_order(nb, 13)).to(dev)
    if producers == 0:
        recv = peer_src.to(dev)
        for i, j in enumerate(others):
            C_final[j * s:(j + 1) * s] = reduced[i].to(dev)
        flags = torch.full((nb,), 4, dtype=torch.int32, device=dev)
    else:
        recv = torch.zeros_like(peer_src, device=dev)
        flags = torch.zeros(nb, dtype=torch.int32, device=dev)
    ops.gemm_ar_two_shot(A.to(dev), B.to(dev), C_final, sends, peer_src.to(dev), recv, reduced.to(dev), world, rank,
                         flags, order, epoch=4, num_producers=producers, num_cus=num_cus, stage_counters=counters,
                         done_flags=done, spin_limit=4_000_000, error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    Cf = C_final.cpu()
    assert rel_fro(Cf[rank * s:(rank + 1) * s].float(), ref_own) < TOL
    for i, j in enumerate(others):
        assert torch.equal(Cf[j * s:(j + 1) * s], reduced[i]), f"slice {j} not copied exactly"
    mask = torch.ones(M, dtype=torch.bool)
    mask[rank * s:(rank + 1) * s] = False
    assert rel_fro(sends.cpu()[mask].float(), own[mask]) < TOL
    assert (sends.cpu()[~mask] == 0).all()
    assert (flags.cpu() == 4).all()
    tiles_n = N // 256
    own_tiles = [t for t in range(done.numel()) if rank * s <= (t // tiles_n) * 256 < (rank + 1) * s]
    assert (done.cpu()[own_tiles] == 4).all()
    if producers:
        assert torch.equal(recv.cpu(), peer_src)


def test_gemm_ar_equal_partials_known_answer(dev):
    """Every peer partial equal to the own partial => C_final is exactly 8x
    it (integer operands, exact in fp32 and bf16)."""
    M, K, N, world = 512, 128, 512, 8
    g = torch.Generator().manual_seed(5)
    A = torch.randint(-1, 2, (M, K), generator=g).to(torch.bfloat16)
    B = torch.randint(-1, 2, (K, N), generator=g).to(torch.bfloat16)
    P = A.float() @ B.float()
    peers = P.to(torch.bfloat16).unsqueeze(0).repeat(world - 1, 1, 1).contiguous()
    C = torch.zeros((M, N), dtype=torch.bfloat16, device=dev)
    ops.gemm_ar(A.to(dev), B.to(dev), C, None, peers.to(dev), world, None, None, epoch=1, gated=False,
                num_producers=0)
    torch.cuda.synchronize()
    assert torch.equal(C.cpu(), (P * world).to(torch.bfloat16))


def test_mfma_ceiling_probe(dev):
    """The MFMA ceiling probe runs, keeps its work live and reports a clock in
    the board's range; its throughput cannot exceed the published peak at the
    clock it reports (4096 bf16 FLOP per clock per CU)."""
    _say("mfma ceiling probe")
    r = ops.probe_mfma_ceiling(iters=2000, reps=1)
    assert r["finite"]
    assert 0.3 < r["sclk_ghz"] < 3.0
    bound = ops.cu_count() * 4096 * r["sclk_ghz"] * 1e9 / 1e12
    assert 0 < r["tflops"] <= bound * 1.05


@pytest.mark.parametrize("M,N,K,lda", [(256, 32768, 65536, 65536), (256, 256, 32, 1 << 22)])
def test_gemm_rejects_operands_beyond_32bit_windows(dev, M, N, K, lda):
    """B of 4 GiB or more, or a 256-row A tile spanning 2 GiB, is beyond the
    kernel's 32-bit buffer offsets: the call fails with a shape error before
    touching memory (the pointers here are a small real buffer)."""
    from mkernel_amd import capi
    buf = torch.zeros(1024, dtype=torch.bfloat16, device=dev)
    a = capi.GemmArgs(buf.data_ptr(), buf.data_ptr(), buf.data_ptr(), M, N, K, lda, N, N, 0, 256, 0, None, 0)
    rc = capi.lib().mk_gemm(C.byref(a), None)
    assert rc == -2, capi.lib().mk_last_error_string()


@pytest.mark.parametrize("prod", [-1, -2])
def test_ag_gemm_cooperative_staging_full_grid_rounds(dev, prod):
    """The whole grid over several tile rounds (M 16384, N 2048: 512 tiles of
    256 x 256), both cooperative schedules, new stage orders and skipped
    epochs on the same flags and counters: every staged byte and flag exact
    and the result bit-equal to the ungated GEMM."""
    _say(f"ag_gemm cooperative full grid producers={prod}")
    cfg, A, B, _ = _ag_case(dev, shard=2048, K=512, N=2048)
    Ad, Bd = A.to(dev), B.to(dev)
    flags = torch.zeros(cfg.M // 128, dtype=torch.int32, device=dev)
    counters = torch.zeros_like(flags)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    C_ref = torch.empty((cfg.M, cfg.N), dtype=torch.bfloat16, device=dev)
    ops.ag_gemm(None, Ad, Bd, C_ref, None, None, epoch=1, gated=False, num_producers=0)
    for epoch, seed in [(1, 31), (2, 32), (5, 33)]:
        order = torch.from_numpy(wl.stage_order(cfg.M // 128, seed)).to(dev)
        A_full = torch.zeros_like(Ad)
        C = torch.empty_like(C_ref)
        ops.ag_gemm(Ad, A_full, Bd, C, flags, order, epoch=epoch, num_producers=prod, stage_counters=counters,
                    spin_limit=4_000_000, error_word=err)
        torch.cuda.synchronize()
        assert int(err.item()) == 0, "a bounded wait timed out"
        assert torch.equal(A_full, Ad)
        assert (flags == epoch).all()
        assert torch.equal(C, C_ref)
    rows = slice(4096, 4352)
    assert rel_fro(C_ref[rows].float().cpu(), gemm_ref(A[rows], B)) < TOL


@pytest.mark.parametrize("M,N,K,cus,waves", [(2048, 1536, 2048, 32, 8),   # 48 tiles on 32: 16 split 2 ways
                                             (2048, 1536, 2048, 40, 8),   # 8 tail tiles split 4 ways (40 // 8 > 4)
                                             (2048, 1536, 2048, 36, 8),   # 12 tail tiles split 3 ways
                                             (2048, 2560, 1024, 64, 8),   # 80 tiles: 16 split 4 ways
                                             (2048, 1536, 2048, 32, 4),   # 4-wave workgroups, 2-way
                                             (1024, 1024, 4096, 8, 8)])   # 16 tiles on 8: no tail
def test_gemm_split_tail_exchange(dev, M, N, K, cus, waves):
    """K-split tails at capped grids: the 2-way split swaps half tiles
    between its two workgroups, wider splits fold into one owner.  Against
    the oracle, against the unsplit GEMM (fp32 rounding only), identical
    across three launches on one workspace, flags left zeroed."""
    _say(f"gemm split exchange M={M} N={N} K={K} cus={cus} waves={waves}")
    A = wl.randn_bf16((M, K), 31, K ** -0.5).to(dev)
    B = wl.randn_bf16((K, N), 32, K ** -0.5).to(dev)
    ws = torch.zeros(int(ops.capi.lib().mk_query_workspace_bytes(0, M, N, K)), dtype=torch.uint8, device=dev)
    plain = ops.gemm(A, B, tile_m=256, num_cus=cus, waves=waves, split_ws=False)
    outs = [ops.gemm(A, B, tile_m=256, num_cus=cus, waves=waves, split_ws=ws) for _ in range(3)]
    torch.cuda.synchronize()
    ref = gemm_ref(A.cpu(), B.cpu())
    assert rel_fro(outs[0].float().cpu(), ref) < TOL
    assert torch.allclose(outs[0].float(), plain.float(), rtol=2 ** -7, atol=1e-5)
    assert all(torch.equal(outs[0], o) for o in outs[1:])
    assert int(ws[:4096].view(torch.int32).abs().sum()) == 0, "split flags not left zeroed"


def test_gemm_split_tail_exchange_identity_exact(dev):
    """I @ X through a 2-way split tail is exact: each half tile's sum is the
    unsplit sum (products by 0 and 1 are exact in fp32)."""
    n = 2048
    I = torch.eye(n, dtype=torch.bfloat16, device=dev)
    X = wl.randn_bf16((n, 1536), 33).to(dev)
    assert torch.equal(ops.gemm(I, X, tile_m=256, num_cus=32).cpu(), X.cpu())


@pytest.mark.parametrize("prod", [-1, 8, -3])
def test_ag_gemm_graph_replays_device_epoch(dev, prod):
    """AllGather+GEMM recorded once in a HIP graph after mk_epoch_advance,
    reading its epoch from that device word: each replay, with new shard
    contents written between replays (and eager library work and
    synchronizations in between), re-stages the shards under a new epoch and
    gives the ungated GEMM's bits on them.  Waits are bounded."""
    _say(f"ag_gemm graph replays, device epoch, producers={prod}")
    cfg, A, B, order = _ag_case(dev)
    Bd = B.to(dev)
    shards = A.to(dev)
    A_full = torch.zeros_like(shards)
    C = torch.empty((cfg.M, cfg.N), dtype=torch.bfloat16, device=dev)
    flags = torch.zeros(cfg.M // 128, dtype=torch.int32, device=dev)
    counters = torch.zeros_like(flags)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    word = torch.zeros(1, dtype=torch.int32, device=dev)
    od = order.to(dev)

    def step():
        ops.epoch_advance(word)
        ops.ag_gemm(shards, A_full, Bd, C, flags, od, epoch=0, num_producers=prod, stage_counters=counters,
                    spin_limit=4_000_000, error_word=err, epoch_ptr=word)

    step()  # eager: epoch 1
    torch.cuda.synchronize()
    assert int(word.item()) == 1 and (flags.cpu() == 1).all()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    gen = torch.Generator().manual_seed(11)
    for rep in range(4):
        new = (torch.randn(cfg.M, cfg.K, generator=gen) / cfg.K ** 0.5).to(torch.bfloat16)
        shards.copy_(new.to(dev))
        C.fill_(7.0)
        g.replay()
        torch.cuda.synchronize()
        assert int(err.item()) == 0
        epoch = 2 + rep  # the capture itself launched nothing
        assert int(word.item()) == epoch
        assert (flags.cpu() == epoch).all()
        assert torch.equal(A_full.cpu(), new)
        ref = torch.empty_like(C)
        ops.ag_gemm(None, A_full, Bd, ref, None, None, epoch=1, gated=False, num_producers=0)
        torch.cuda.synchronize()
        assert torch.equal(C.cpu(), ref.cpu()), rep


def test_gemm_rs_graph_replays_device_epoch(dev):
    """GEMM+reduce-scatter with cooperative staging in a HIP graph, epoch
    from a device word: every replay with new peer partials folds them (the
    owned slice equals an eager run with a host epoch on the same data)."""
    _say("gemm_rs graph replays, device epoch")
    cfg = wl.RsCfg(world=8, rank=3, M=2048, K=256, N=512)
    A, B, peers, order = wl.rs_inputs(cfg)
    rows = cfg.M // cfg.world
    Ad, Bd, pd = A.to(dev), B.to(dev), peers.to(dev)
    nfl = (cfg.world - 1) * rows // 128
    od = torch.from_numpy(order).to(dev)
    work = torch.zeros((cfg.M, cfg.N), dtype=torch.bfloat16, device=dev)
    out = torch.zeros((rows, cfg.N), dtype=torch.bfloat16, device=dev)
    recv = torch.zeros_like(pd)
    flags = torch.zeros(nfl, dtype=torch.int32, device=dev)
    counters = torch.zeros_like(flags)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    word = torch.zeros(1, dtype=torch.int32, device=dev)

    def step():
        ops.epoch_advance(word)
        ops.gemm_rs(Ad, Bd, work, out, pd, recv, cfg.world, cfg.rank, flags, od, epoch=0, num_producers=-1,
                    stage_counters=counters, spin_limit=4_000_000, error_word=err, epoch_ptr=word)

    step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    gen = torch.Generator().manual_seed(12)
    e_flags = torch.zeros_like(flags)
    e_counters = torch.zeros_like(flags)
    for rep in range(3):
        new = (torch.randn(peers.shape, generator=gen) * 0.5).to(torch.bfloat16)
        pd.copy_(new.to(dev))
        out.fill_(5.0)
        g.replay()
        torch.cuda.synchronize()
        assert int(err.item()) == 0 and (flags.cpu() == 2 + rep).all()
        assert torch.equal(recv.cpu(), new)
        ref = torch.zeros_like(out)
        ops.gemm_rs(Ad, Bd, torch.zeros_like(work), ref, pd, torch.zeros_like(recv), cfg.world, cfg.rank, e_flags, od,
                    epoch=1 + rep, num_producers=-1, stage_counters=e_counters)
        torch.cuda.synchronize()
        assert torch.equal(out.cpu(), ref.cpu()), rep


def test_gemm_ar_graph_replays_device_epoch(dev):
    """GEMM + all-reduce in a HIP graph after mk_epoch_advance: each replay
    with new peer partials stages them under a new epoch, publishes every
    tile's done flag with it, and gives the bits of an eager launch with a
    host epoch on the same data."""
    _say("gemm_ar graph replays, device epoch")
    world, M, N, K = 8, 512, 512, 256
    A = wl.randn_bf16((M, K), 40, K ** -0.5).to(dev)
    B = wl.randn_bf16((K, N), 41, K ** -0.5).to(dev)
    peers = wl.randn_bf16((world - 1, M, N), 42, 0.5).to(dev)
    nflags = (world - 1) * M // 128
    ntiles = (M // 256) * (N // 256)
    order = torch.from_numpy(wl.stage_order(nflags, 3)).to(dev)
    recv = torch.zeros_like(peers)
    flags = torch.zeros(nflags, dtype=torch.int32, device=dev)
    counters = torch.zeros_like(flags)
    done = torch.zeros(ntiles, dtype=torch.int32, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    word = torch.zeros(1, dtype=torch.int32, device=dev)
    C = torch.empty((M, N), dtype=torch.bfloat16, device=dev)

    def step():
        ops.epoch_advance(word)
        ops.gemm_ar(A, B, C, peers, recv, world, flags, order, epoch=0, num_producers=-1, stage_counters=counters,
                    done_flags=done, spin_limit=4_000_000, error_word=err, epoch_ptr=word)

    step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    gen = torch.Generator().manual_seed(13)
    e_flags, e_counters, e_done = torch.zeros_like(flags), torch.zeros_like(flags), torch.zeros_like(done)
    for rep in range(3):
        new = (torch.randn(peers.shape, generator=gen) * 0.5).to(torch.bfloat16)
        peers.copy_(new.to(dev))
        C.fill_(3.0)
        g.replay()
        torch.cuda.synchronize()
        epoch = 2 + rep
        assert int(err.item()) == 0
        assert (flags.cpu() == epoch).all() and (done.cpu() == epoch).all()
        assert torch.equal(recv.cpu(), new)
        ref = torch.empty_like(C)
        ops.gemm_ar(A, B, ref, peers, torch.zeros_like(recv), world, e_flags, order, epoch=1 + rep,
                    num_producers=-1, stage_counters=e_counters, done_flags=e_done)
        torch.cuda.synchronize()
        assert torch.equal(C.cpu(), ref.cpu()), rep


def test_grid_larger_than_device_is_refused(dev):
    """Every workgroup of a persistent launch must be resident (flag waits,
    cooperative staging and the K-split exchange wait on each other): a grid
    above the CU count is refused before any launch."""
    _say("grid > CUs refused")
    cus = ops.cu_count()
    A = torch.zeros((256, 256), dtype=torch.bfloat16, device=dev)
    with pytest.raises(MkError, match="num_cus"):
        ops.gemm(A, A, num_cus=cus + 8)
    C = torch.empty_like(A)
    flags = torch.zeros(2, dtype=torch.int32, device=dev)
    with pytest.raises(MkError, match="num_cus"):
        ops.ag_gemm(A, A, A, C, flags, None, epoch=1, num_cus=cus + 1, stage_counters=torch.zeros_like(flags))
    with pytest.raises(MkError, match="num_cus"):
        ops.gemm_rs(A, A, C, C, None, None, 1, 0, None, None, epoch=1, gated=False, num_cus=2 * cus)
    with pytest.raises(MkError, match="num_cus"):
        ops.gemm_ar(A, A, C, None, None, 1, None, None, epoch=1, gated=False, num_cus=cus + 1)
    rbe = torch.zeros(2, dtype=torch.int32, device=dev)
    with pytest.raises(MkError, match="num_cus"):
        ops.moe_grouped_gemm(A, A.view(1, 256, 256), C, rb_expert=rbe, num_cus=cus + 1)
    torch.cuda.synchronize()


@pytest.mark.parametrize("world,rank", [(8, 3), (8, 0)])
def test_ag_gemm_present_blocks_not_copied(dev, world, rank):
    """n_present: the first stage positions name blocks already in A_full
    (the own shard); their flags are published, their source rows are never
    read (junk there must not reach A_full or C)."""
    _say(f"ag n_present world={world} rank={rank}")
    cfg = wl.AgCfg(world=world, shard_rows=256, K=512, N=512)
    A, B, order = wl.ag_inputs(cfg)
    nb, per = cfg.M // 128, cfg.shard_rows // 128
    own = list(range(rank * per, (rank + 1) * per))
    full_order = torch.tensor(own + [int(b) for b in order if int(b) not in own], dtype=torch.int32, device=dev)
    src = A.clone()
    src[rank * cfg.shard_rows:(rank + 1) * cfg.shard_rows] = float("nan")
    A_full = torch.zeros_like(A)
    A_full[rank * cfg.shard_rows:(rank + 1) * cfg.shard_rows] = A[rank * cfg.shard_rows:(rank + 1) * cfg.shard_rows]
    A_full = A_full.to(dev)
    flags = torch.zeros(nb, dtype=torch.int32, device=dev)
    counters = torch.zeros_like(flags)
    C = torch.empty((cfg.M, cfg.N), dtype=torch.bfloat16, device=dev)
    for epoch, prod in ((1, -1), (2, -2), (3, 4), (4, -3)):
        ops.ag_gemm(src.to(dev), A_full, B.to(dev), C, flags, full_order, epoch=epoch, num_producers=prod,
                    stage_counters=counters, n_present=per)
        torch.cuda.synchronize()
        assert torch.equal(A_full.cpu(), A)
        assert (flags.cpu() == epoch).all()
        assert rel_fro(C.float(), ag_gemm_ref(A, B)) < TOL
