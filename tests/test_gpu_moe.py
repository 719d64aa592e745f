"""GPU parity of the MoE expert path (permute, grouped GEMM1 [+SwiGLU],
GEMM2, combine) against the CPU oracle, through the C-ABI."""
import numpy as np
import pytest
import torch

from mkernel_amd import ops, workloads as wl
from oracle import moe as om
from oracle.gemm import rel_fro

pytestmark = pytest.mark.gpu
TOL = 2e-2

SMALL = wl.MoeCfg(tokens=512, H=512, I=256, experts=64, topk=8, ep=8, rank=1)


def _say(msg):
    print(msg, flush=True)


def _setup(dev, cfg=SMALL):
    tokens, ids, gates, w1, w2 = wl.moe_inputs(cfg)
    idx = ops.moe_build_indices(ids, gates, cfg.e0, cfg.n_local)
    d = {k: torch.from_numpy(np.ascontiguousarray(v)).to(dev) for k, v in idx.items() if isinstance(v, np.ndarray)}
    return tokens, ids, gates, w1, w2, idx, d


def test_permute_bit_exact(dev):
    _say("moe permute")
    tokens, ids, gates, w1, w2, idx, d = _setup(dev)
    post = torch.full((idx["R_pad"], SMALL.H), 7.0, dtype=torch.bfloat16, device=dev)
    ops.moe_permute(tokens.to(dev), d["pull_indices"], post)
    torch.cuda.synchronize()
    assert torch.equal(post.cpu(), om.permute_ref(tokens, idx["pull_indices"]))


@pytest.mark.parametrize("tile_n", [256, 512])
@pytest.mark.parametrize("split", [None, False])
@pytest.mark.parametrize("use_rb,skip_pad", [(True, False), (False, False), (True, True)])
def test_grouped_gemm1(dev, use_rb, skip_pad, split, tile_n):
    """split None: the tail round is K-split through the default workspace;
    False: no K-split."""
    _say(f"moe grouped gemm1 use_rb={use_rb} skip_pad={skip_pad} split={split} tile_n={tile_n}")
    tokens, ids, gates, w1, w2, idx, d = _setup(dev)
    post = om.permute_ref(tokens, idx["pull_indices"])
    out = torch.full((idx["R_pad"], 2 * SMALL.I), 3.0, dtype=torch.bfloat16, device=dev)
    ops.moe_grouped_gemm(post.to(dev), w1.to(dev), out, rb_expert=d["rb_expert"] if use_rb else None,
                         padded_tokens_per_expert=None if use_rb else d["padded_tokens_per_expert"], mode=0,
                         rb_rows=d["rb_rows"] if skip_pad else None, split_ws=split, tile_n=tile_n)
    torch.cuda.synchronize()
    ref = om.grouped_gemm_ref(post, w1, idx["padded_tokens_per_expert"])
    assert rel_fro(out.float(), ref) < TOL
    pad = idx["pull_indices"][:, 0] < 0
    assert (out.cpu()[torch.from_numpy(pad)] == 0).all()  # zero rows stay zero


MANY = wl.MoeCfg(tokens=1024, H=256, I=2304, experts=64, topk=8, ep=8, rank=0)


@pytest.mark.parametrize("split", [None, False])
def test_grouped_gemm_many_column_tiles(dev, split):
    """More than 8 column tiles and no epilogue (GEMM2's shape class: 9 or
    18 column tiles here), where the tiles walk each expert's run of row
    tiles together, including a multi-tile expert: every row matches the
    oracle, padding rows stay zero, and without a K-split both tile widths
    give the same bits."""
    _say(f"moe grouped gemm, many column tiles, split={split}")
    tokens, ids, gates, w1, w2, idx, d = _setup(dev, MANY)
    assert (idx["padded_tokens_per_expert"] > 128).any()  # some expert spans several row tiles
    post = om.permute_ref(tokens, idx["pull_indices"])
    outs = []
    for tile_n in (512, 256):
        out = torch.full((idx["R_pad"], 2 * MANY.I), 3.0, dtype=torch.bfloat16, device=dev)
        ops.moe_grouped_gemm(post.to(dev), w1.to(dev), out, rb_expert=d["rb_expert"], mode=0,
                             rb_rows=d["rb_rows"], split_ws=split, tile_n=tile_n)
        torch.cuda.synchronize()
        outs.append(out.cpu())
    ref = om.grouped_gemm_ref(post, w1, idx["padded_tokens_per_expert"])
    pad = torch.from_numpy(idx["pull_indices"][:, 0] < 0)
    for out in outs:
        assert rel_fro(out.float(), ref) < TOL
        assert (out[pad] == 0).all()
    if split is False:
        assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("tile_n", [256, 512])
@pytest.mark.parametrize("split", [None, False])
def test_gemm1_swiglu(dev, split, tile_n):
    _say(f"moe gemm1+swiglu split={split} tile_n={tile_n}")
    tokens, ids, gates, w1, w2, idx, d = _setup(dev)
    post = om.permute_ref(tokens, idx["pull_indices"])
    act = torch.empty((idx["R_pad"], SMALL.I), dtype=torch.bfloat16, device=dev)
    ops.moe_grouped_gemm(post.to(dev), w1.to(dev), act, rb_expert=d["rb_expert"], mode=1, split_ws=split,
                         tile_n=tile_n)
    torch.cuda.synchronize()
    ref_act, _ = om.ffn_ref(post, w1, w2, idx["padded_tokens_per_expert"], SMALL.I)
    assert rel_fro(act.float(), ref_act) < TOL


WIDE = wl.MoeCfg(tokens=512, H=1024, I=512, experts=64, topk=8, ep=8, rank=1)


@pytest.mark.parametrize("mode", [0, 1])
def test_tile_widths_bit_identical(dev, mode):
    """Without a K-split every output element is accumulated over the same K
    stages in the same order by the 128x256 and the 128x512 tiles, so the two
    widths give the same bits (pins the wide tile's B staging, SwiGLU column
    pairing and store addressing against the narrow one)."""
    _say(f"moe tile widths mode={mode}")
    tokens, ids, gates, w1, w2, idx, d = _setup(dev, WIDE)
    post = om.permute_ref(tokens, idx["pull_indices"]).to(dev)
    ncol = 2 * WIDE.I if mode == 0 else WIDE.I
    outs = []
    for tn in (256, 512):
        out = torch.full((idx["R_pad"], ncol), 5.0, dtype=torch.bfloat16, device=dev)
        ops.moe_grouped_gemm(post, w1.to(dev), out, rb_expert=d["rb_expert"], mode=mode, rb_rows=d["rb_rows"],
                             split_ws=False, tile_n=tn)
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.equal(outs[0].cpu(), outs[1].cpu())
    ref_act, _ = om.ffn_ref(post.cpu(), w1, w2, idx["padded_tokens_per_expert"], WIDE.I)
    ref = ref_act if mode == 1 else om.grouped_gemm_ref(post.cpu(), w1, idx["padded_tokens_per_expert"])
    assert rel_fro(outs[1].float(), ref) < TOL


def test_grouped_gemm_tile_n_rejected(dev):
    tokens, ids, gates, w1, w2, idx, d = _setup(dev)
    post = om.permute_ref(tokens, idx["pull_indices"]).to(dev)
    out = torch.empty((idx["R_pad"], SMALL.H), dtype=torch.bfloat16, device=dev)
    w = torch.zeros((SMALL.n_local, SMALL.I, 768), dtype=torch.bfloat16, device=dev)
    with pytest.raises(RuntimeError):
        ops.moe_grouped_gemm(post[:, :SMALL.I].contiguous(), w, torch.empty((idx["R_pad"], 768), dtype=torch.bfloat16,
                             device=dev), rb_expert=d["rb_expert"], tile_n=512)
    with pytest.raises(RuntimeError):
        ops.moe_grouped_gemm(post, w1.to(dev), out, rb_expert=d["rb_expert"], tile_n=384)


def test_combine(dev):
    _say("moe combine")
    tokens, ids, gates, w1, w2, idx, d = _setup(dev)
    ye = wl.randn_bf16((idx["R_pad"], SMALL.H), 21)
    for dtype in (torch.float32, torch.bfloat16):
        y = torch.empty((SMALL.tokens, SMALL.H), dtype=dtype, device=dev)
        ops.moe_combine(ye.to(dev), d["row_weight"], d["owner_offset"], d["slot_to_row"], y)
        torch.cuda.synchronize()
        ref = om.combine_ref(ye, idx["row_weight"], idx["pull_indices"], SMALL.tokens)
        assert rel_fro(y.float(), ref) < (1e-6 if dtype == torch.float32 else 1e-2)


def test_tile_rows_bit_exact(dev):
    tokens, ids, gates, w1, w2, idx, d = _setup(dev)
    rb = torch.full((idx["R_pad"] // 128,), -1, dtype=torch.int32, device=dev)
    ops.moe_tile_rows(d["pull_indices"], rb)
    torch.cuda.synchronize()
    assert np.array_equal(rb.cpu().numpy(), idx["rb_rows"])
    assert np.array_equal(idx["rb_rows"], om.build_indices_np(ids, gates, SMALL.e0, SMALL.n_local)["rb_rows"])


def test_invert_slots_bit_exact(dev):
    tokens, ids, gates, w1, w2, idx, d = _setup(dev)
    s2r = torch.full((idx["R"],), -5, dtype=torch.int32, device=dev)
    ops.moe_invert_slots(d["row_to_slot"], d["row_to_owner"], s2r)
    torch.cuda.synchronize()
    assert np.array_equal(s2r.cpu().numpy(), idx["slot_to_row"])


def test_invert_slots_owner_and_capacity(dev):
    """Rows of another owner are left out, slots past the capacity are not
    written and are reported, every other entry ends at -1 (the combine
    skips those slots)."""
    _say("moe invert slots owner / capacity")
    r2s = torch.tensor([3, 0, 7, 1, 2, 9, 0], dtype=torch.int32, device=dev)
    own = torch.tensor([0, 0, 1, 0, -1, 0, 0], dtype=torch.int32, device=dev)
    s2r = torch.full((5,), 123, dtype=torch.int32, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    ops.moe_invert_slots(r2s[:6], own[:6], s2r, owner=0, error_word=err)
    torch.cuda.synchronize()
    # row 2 belongs to owner 1, row 4 is padding, row 5's slot 9 is past the capacity 5
    assert s2r.cpu().tolist() == [1, 3, -1, 0, -1]
    assert int(err.item()) == 2
    err.zero_()
    ops.moe_invert_slots(r2s[:6], own[:6], s2r, owner=1, error_word=err)
    torch.cuda.synchronize()
    assert s2r.cpu().tolist() == [-1, -1, -1, -1, -1] and int(err.item()) == 2  # slot 7 of owner 1 is past it too


def test_combine_skips_unproduced_slots(dev):
    """A slot whose row stays -1 (produced on another GPU) adds nothing."""
    _say("moe combine skips -1 slots")
    H = 256
    ye = wl.randn_bf16((4, H), 3, 1.0).to(dev)
    w = torch.tensor([0.5, 2.0, 1.0, 3.0], dtype=torch.float32, device=dev)
    off = torch.tensor([0, 2, 3], dtype=torch.int32, device=dev)
    s2r = torch.tensor([1, -1, 3], dtype=torch.int32, device=dev)
    y = torch.full((2, H), 9.0, dtype=torch.float32, device=dev)
    ops.moe_combine(ye, w, off, s2r, y)
    torch.cuda.synchronize()
    yf = ye.float().cpu()
    assert torch.equal(y.cpu()[0], 2.0 * yf[1])
    assert torch.equal(y.cpu()[1], 3.0 * yf[3])


@pytest.mark.parametrize("tile_n", [0, 256])
def test_ffn_combine_end_to_end(dev, tile_n):
    _say(f"moe ffn+combine tile_n={tile_n}")
    tokens, ids, gates, w1, w2, idx, d = _setup(dev)
    R_pad = idx["R_pad"]
    post = torch.empty((R_pad, SMALL.H), dtype=torch.bfloat16, device=dev)
    act = torch.empty((R_pad, SMALL.I), dtype=torch.bfloat16, device=dev)
    ye = torch.empty((R_pad, SMALL.H), dtype=torch.bfloat16, device=dev)
    y = torch.empty((SMALL.tokens, SMALL.H), dtype=torch.bfloat16, device=dev)
    ops.moe_ffn_combine(tokens.to(dev), d["pull_indices"], d["row_weight"], d["owner_offset"], d["slot_to_row"],
                        w1.to(dev), w2.to(dev), post, act, ye, y, rb_expert=d["rb_expert"], rb_rows=d["rb_rows"],
                        tile_n=tile_n)
    torch.cuda.synchronize()
    post_ref = om.permute_ref(tokens, idx["pull_indices"])
    assert torch.equal(post.cpu(), post_ref)
    _, ye_ref = om.ffn_ref(post_ref, w1, w2, idx["padded_tokens_per_expert"], SMALL.I)
    assert rel_fro(ye.float(), ye_ref) < TOL
    y_ref = om.combine_ref(ye_ref, idx["row_weight"], idx["pull_indices"], SMALL.tokens)
    assert rel_fro(y.float(), y_ref) < TOL
    # determinism: a second run is byte-identical
    y2 = torch.empty_like(y)
    ops.moe_ffn_combine(tokens.to(dev), d["pull_indices"], d["row_weight"], d["owner_offset"], d["slot_to_row"],
                        w1.to(dev), w2.to(dev), post, act, ye, y2, rb_expert=d["rb_expert"], tile_n=tile_n)
    torch.cuda.synchronize()
    assert torch.equal(y.cpu(), y2.cpu())


@pytest.mark.parametrize("mode", [0, 1])
def test_fused_dispatch_gemm_matches_permute(dev, mode):
    """GEMM1 gathering its rows through the pull table (fused dispatch) is
    bit-identical to permute + GEMM1 (the same bytes reach the MFMAs)."""
    _say(f"moe fused dispatch mode={mode}")
    tokens, ids, gates, w1, w2, idx, d = _setup(dev)
    Rp = idx["R_pad"]
    post = torch.empty((Rp, SMALL.H), dtype=torch.bfloat16, device=dev)
    ops.moe_permute(tokens.to(dev), d["pull_indices"], post)
    ncol = 2 * SMALL.I if mode == 0 else SMALL.I
    ref = torch.empty((Rp, ncol), dtype=torch.bfloat16, device=dev)
    out = torch.full((Rp, ncol), 5.0, dtype=torch.bfloat16, device=dev)
    ops.moe_grouped_gemm(post, w1.to(dev), ref, rb_expert=d["rb_expert"], mode=mode, rb_rows=d["rb_rows"])
    ops.moe_grouped_gemm(tokens.to(dev), w1.to(dev), out, rb_expert=d["rb_expert"], mode=mode, rb_rows=d["rb_rows"],
                         gather_pull=d["pull_indices"])
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), ref.cpu())


def test_fused_dispatch_multi_source(dev):
    """Pull rows naming other source devices/nodes: token row
    (src_node * devs + src_dev) * tokens_per_src + src_token."""
    _say("moe fused dispatch multi-source")
    g = torch.Generator().manual_seed(9)
    tps, devs, nodes, K, N = 40, 2, 2, 256, 256
    src = wl.randn_bf16((nodes * devs * tps, K), 31)
    Rp = 256
    pull = torch.full((Rp, 3), -1, dtype=torch.int32)
    real = 200
    pull[:real, 0] = torch.randint(0, nodes, (real,), generator=g)
    pull[:real, 1] = torch.randint(0, devs, (real,), generator=g)
    pull[:real, 2] = torch.randint(0, tps, (real,), generator=g)
    w = wl.randn_bf16((2, K, N), 32, K ** -0.5)
    rb_expert = torch.tensor([0, 1], dtype=torch.int32)
    post_ref = om.permute_ref(src, pull.numpy(), tokens_per_src=tps, devs_per_node=devs)
    post = torch.empty((Rp, K), dtype=torch.bfloat16, device=dev)
    ops.moe_permute(src.to(dev), pull.to(dev), post, tokens_per_src=tps, devs_per_node=devs)
    assert torch.equal(post.cpu(), post_ref)
    ref = torch.empty((Rp, N), dtype=torch.bfloat16, device=dev)
    out = torch.empty((Rp, N), dtype=torch.bfloat16, device=dev)
    ops.moe_grouped_gemm(post, w.to(dev), ref, rb_expert=rb_expert.to(dev))
    ops.moe_grouped_gemm(src.to(dev), w.to(dev), out, rb_expert=rb_expert.to(dev), gather_pull=pull.to(dev),
                         tokens_per_src=tps, devs_per_node=devs)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), ref.cpu())
    # spot-check one routed row against the oracle matmul
    r = 7
    srow = (int(pull[r, 0]) * devs + int(pull[r, 1])) * tps + int(pull[r, 2])
    exp = src[srow].float() @ w[0].float()
    assert rel_fro(out[r].cpu().float()[None], exp[None]) < TOL


def test_ffn_combine_fused_dispatch_bit_identical(dev):
    _say("moe ffn+combine fused dispatch")
    tokens, ids, gates, w1, w2, idx, d = _setup(dev)
    Rp = idx["R_pad"]
    ys = []
    for fuse in (False, True):
        post = None if fuse else torch.empty((Rp, SMALL.H), dtype=torch.bfloat16, device=dev)
        act = torch.empty((Rp, SMALL.I), dtype=torch.bfloat16, device=dev)
        ye = torch.empty((Rp, SMALL.H), dtype=torch.bfloat16, device=dev)
        y = torch.empty((SMALL.tokens, SMALL.H), dtype=torch.float32, device=dev)
        ops.moe_ffn_combine(tokens.to(dev), d["pull_indices"], d["row_weight"], d["owner_offset"], d["slot_to_row"],
                            w1.to(dev), w2.to(dev), post, act, ye, y, rb_expert=d["rb_expert"], rb_rows=d["rb_rows"],
                            fuse_dispatch=fuse)
        ys.append(y.cpu())
    assert torch.equal(ys[0], ys[1])


@pytest.mark.parametrize("fuse", [False, True])
def test_ffn_combine_no_local_rows(dev, fuse):
    """A rank that no token routes to: R_pad = 0, every table empty; the
    layer writes y = 0 and launches no GEMM."""
    _say(f"moe ffn no local rows fuse={fuse}")
    cfg = wl.MoeCfg(tokens=64, H=512, I=256, experts=64, topk=4, ep=8, rank=1)
    tokens, ids, gates, w1, w2 = wl.moe_inputs(cfg)
    ids = np.where((ids >= cfg.e0) & (ids < cfg.e0 + cfg.n_local), 0, ids)  # expert 0 belongs to rank 0
    idx = ops.moe_build_indices(ids, gates, cfg.e0, cfg.n_local)
    assert idx["R"] == 0 and idx["R_pad"] == 0
    d = {k: torch.from_numpy(np.ascontiguousarray(v)).to(dev) for k, v in idx.items() if isinstance(v, np.ndarray)}
    empty = torch.empty((0, cfg.H), dtype=torch.bfloat16, device=dev)
    act = torch.empty((0, cfg.I), dtype=torch.bfloat16, device=dev)
    y = torch.full((cfg.tokens, cfg.H), 9.0, dtype=torch.float32, device=dev)
    ops.moe_ffn_combine(tokens.to(dev), d["pull_indices"], d["row_weight"], d["owner_offset"], d["slot_to_row"],
                        w1.to(dev), w2.to(dev), None if fuse else empty, act, empty, y, rb_expert=d["rb_expert"],
                        rb_rows=d["rb_rows"], fuse_dispatch=fuse)
    torch.cuda.synchronize()
    assert (y.cpu() == 0).all()
    # the single-stage entries accept the empty tables too
    ops.moe_permute(tokens.to(dev), d["pull_indices"], empty)
    ops.moe_grouped_gemm(empty, w1.to(dev), act, rb_expert=d["rb_expert"], mode=1)
    ops.moe_tile_rows(d["pull_indices"], torch.empty((0,), dtype=torch.int32, device=dev))
    ops.moe_invert_slots(d["row_to_slot"], d["row_to_owner"], torch.empty((0,), dtype=torch.int32, device=dev))
    torch.cuda.synchronize()


def test_ffn_combine_ragged_extremes(dev):
    """One token sends all top-k choices to local experts (one of them
    twice), most tokens send none: slots, padding and the combine handle
    both ends."""
    _say("moe ffn ragged extremes")
    cfg = wl.MoeCfg(tokens=256, H=512, I=256, experts=64, topk=8, ep=8, rank=2)
    tokens, ids, gates, w1, w2 = wl.moe_inputs(cfg)
    local = (ids >= cfg.e0) & (ids < cfg.e0 + cfg.n_local)
    ids = np.where(local, (ids + cfg.n_local) % cfg.experts, ids)  # route everything away...
    ids[7] = cfg.e0 + np.array([0, 1, 2, 3, 4, 5, 6, 6])           # ...except token 7
    ids[200, :2] = cfg.e0 + 3                                       # and two entries of token 200
    idx = ops.moe_build_indices(ids, gates, cfg.e0, cfg.n_local)
    assert idx["R"] == 10
    d = {k: torch.from_numpy(np.ascontiguousarray(v)).to(dev) for k, v in idx.items() if isinstance(v, np.ndarray)}
    R_pad = idx["R_pad"]
    act = torch.empty((R_pad, cfg.I), dtype=torch.bfloat16, device=dev)
    ye = torch.empty((R_pad, cfg.H), dtype=torch.bfloat16, device=dev)
    y = torch.full((cfg.tokens, cfg.H), 9.0, dtype=torch.float32, device=dev)
    ops.moe_ffn_combine(tokens.to(dev), d["pull_indices"], d["row_weight"], d["owner_offset"], d["slot_to_row"],
                        w1.to(dev), w2.to(dev), None, act, ye, y, rb_expert=d["rb_expert"], rb_rows=d["rb_rows"],
                        fuse_dispatch=True)
    torch.cuda.synchronize()
    post = om.permute_ref(tokens, idx["pull_indices"])
    _, ye_ref = om.ffn_ref(post, w1, w2, idx["padded_tokens_per_expert"], cfg.I)
    y_ref = om.combine_ref(ye_ref, idx["row_weight"], idx["pull_indices"], cfg.tokens)
    assert rel_fro(y.float().cpu(), y_ref) < TOL
    routed = torch.zeros(cfg.tokens, dtype=torch.bool)
    routed[[7, 200]] = True
    assert (y.cpu()[~routed] == 0).all()


@pytest.mark.parametrize("tile_n", [256, 512])
def test_swiglu_epilogue_values(dev, tile_n):
    """The SwiGLU epilogue on exactly known gate/up values: one-hot rows of A
    select rows of one expert's W1, so h = W1 rows exactly and act must be
    bf16(silu(g) * u) of those bf16 values, including large gates (e^-g
    overflows to inf: silu -> -0 / silu -> g), zero and tiny gates.  Every
    element within one bf16 rounding step of the fp32 oracle."""
    _say(f"moe swiglu epilogue values tile_n={tile_n}")
    K, I = 128, 512
    g = torch.linspace(-100.0, 100.0, K * I).reshape(K, I)
    g[:, :8] = torch.tensor([0.0, -0.0, 1e-30, -1e-30, 88.0, -88.0, 1e4, -1e4])
    u = wl.randn_bf16((K, I), 41).float()
    w1 = torch.cat([g, u], dim=1).to(torch.bfloat16).unsqueeze(0)  # [1, K, 2I]
    A = torch.zeros((128, K), dtype=torch.bfloat16)
    A[torch.arange(128), torch.arange(128) % K] = 1.0
    rb_expert = torch.zeros(1, dtype=torch.int32, device=dev)
    act = torch.empty((128, I), dtype=torch.bfloat16, device=dev)
    ops.moe_grouped_gemm(A.to(dev), w1.to(dev), act, rb_expert=rb_expert, mode=1, split_ws=False, tile_n=tile_n)
    torch.cuda.synchronize()
    ref = om.silu_mul(w1[0, :, :I].float(), w1[0, :, I:].float())
    got = act.cpu().float()
    assert torch.isfinite(got).all()
    assert torch.allclose(got, ref, rtol=2 ** -7, atol=1e-30)


def test_gemm1_swiglu_split_tail_exchange(dev):
    """Grouped GEMM1 + SwiGLU with a capped grid so the tail round is split
    2 ways (half-tile swap): against the oracle, bit-equal across repeated
    launches, and within rounding of the unsplit launch."""
    _say("moe gemm1+swiglu split exchange")
    tokens, ids, gates, w1, w2, idx, d = _setup(dev, WIDE)
    post = om.permute_ref(tokens, idx["pull_indices"])
    ntiles = (idx["R_pad"] // 128) * (2 * WIDE.I // 512)
    # a grid whose tail (ntiles % cus tiles) the library splits 2 ways: cus / tail in [2, 3)
    cus = next(c for c in range(2, ntiles) if ntiles % c and 2 <= c // (ntiles % c) < 3)
    outs = []
    for split in (None, None, False):
        act = torch.empty((idx["R_pad"], WIDE.I), dtype=torch.bfloat16, device=dev)
        ops.moe_grouped_gemm(post.to(dev), w1.to(dev), act, rb_expert=d["rb_expert"], mode=1, split_ws=split,
                             tile_n=512, num_cus=cus)
        outs.append(act)
    torch.cuda.synchronize()
    ref_act, _ = om.ffn_ref(post, w1, w2, idx["padded_tokens_per_expert"], WIDE.I)
    assert rel_fro(outs[0].float().cpu(), ref_act) < TOL
    assert torch.equal(outs[0], outs[1])
    assert torch.allclose(outs[0].float(), outs[2].float(), rtol=2 ** -6, atol=1e-3)


def test_ffn_combine_random_layers(dev):
    """Seeded random MoE layers: token count, hidden and FFN widths, expert
    count, top-k, expert-parallel size, rank, routing skew, fused or separate
    dispatch, tile width.  y_expert and y match the oracle, rows the rank
    does not route stay zero, and a second run is byte-identical."""
    rng = np.random.default_rng(1234)
    for case in range(8):
        experts = int(rng.choice([16, 32, 64]))
        ep = int(rng.choice([1, 2, 4, 8]))
        cfg = wl.MoeCfg(tokens=int(rng.integers(1, 9)) * 96, H=int(rng.integers(1, 5)) * 256,
                        I=int(rng.integers(1, 5)) * 128, experts=experts, topk=int(rng.integers(1, 9)), ep=ep,
                        rank=int(rng.integers(0, ep)), zipf_s=float(rng.choice([0.0, 1.1, 2.0])))
        fuse = bool(rng.integers(0, 2))
        tile_n = int(rng.choice([0, 256]))
        _say(f"moe random case={case} {cfg} fuse={fuse} tile_n={tile_n}")
        tokens, ids, gates, w1, w2 = wl.moe_inputs(cfg, seed=500 + case)
        idx = ops.moe_build_indices(ids, gates, cfg.e0, cfg.n_local)
        d = {k: torch.from_numpy(np.ascontiguousarray(v)).to(dev) for k, v in idx.items()
             if isinstance(v, np.ndarray)}
        R_pad = idx["R_pad"]
        post = None if fuse else torch.empty((R_pad, cfg.H), dtype=torch.bfloat16, device=dev)
        act = torch.empty((R_pad, cfg.I), dtype=torch.bfloat16, device=dev)
        ye = torch.empty((R_pad, cfg.H), dtype=torch.bfloat16, device=dev)
        ys = []
        for _ in range(2):
            y = torch.full((cfg.tokens, cfg.H), 7.0, dtype=torch.float32, device=dev)
            ops.moe_ffn_combine(tokens.to(dev), d["pull_indices"], d["row_weight"], d["owner_offset"],
                                d["slot_to_row"], w1.to(dev), w2.to(dev), post, act, ye, y,
                                rb_expert=d["rb_expert"], rb_rows=d["rb_rows"], fuse_dispatch=fuse, tile_n=tile_n)
            torch.cuda.synchronize()
            ys.append(y.cpu())
        assert torch.equal(ys[0], ys[1]), f"case {case}: not deterministic"
        post_ref = om.permute_ref(tokens, idx["pull_indices"])
        _, ye_ref = om.ffn_ref(post_ref, w1, w2, idx["padded_tokens_per_expert"], cfg.I)
        y_ref = om.combine_ref(ye_ref, idx["row_weight"], idx["pull_indices"], cfg.tokens)
        if idx["R"] > 0:
            real = torch.from_numpy(np.asarray(idx["pull_indices"])[:, 2] >= 0)
            assert rel_fro(ye.cpu().float()[real], ye_ref[real]) < TOL, f"case {case}: y_expert"
            assert rel_fro(ys[0], y_ref) < TOL, f"case {case}: y"
        routed = torch.from_numpy(np.diff(np.asarray(idx["owner_offset"])) > 0)
        assert (ys[0][~routed] == 0).all(), f"case {case}: unrouted tokens"
