"""GPU routing-index build (mk_moe_build_indices_dev) against the host
builder mk_moe_build_indices, table by table and bit for bit.  The host
builder is itself pinned to the oracle's restatements of the reference's
Python builders (tests/test_capi_host.py, tests/test_oracle.py)."""
import numpy as np
import pytest
import torch

from mkernel_amd import ops, workloads as wl

pytestmark = pytest.mark.gpu

TABLES = ("padded_tokens_per_expert", "local_rb_per_expert", "pull_indices", "row_expert", "rb_expert", "rb_rows",
          "row_weight", "owner_offset", "row_to_slot", "row_to_owner", "slot_to_row")


def _say(msg):
    print(msg, flush=True)


def _check(dev, ids, gates, e0, n_local, row_block=128):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    gates = np.ascontiguousarray(gates, dtype=np.float32)
    host = ops.moe_build_indices(ids, gates, e0, n_local, row_block)
    gpu = ops.moe_build_indices_dev(torch.from_numpy(ids).to(dev), torch.from_numpy(gates).to(dev), e0, n_local,
                                    row_block)
    assert (gpu["R"], gpu["R_pad"]) == (host["R"], host["R_pad"])
    for f in TABLES:
        h = np.asarray(host[f])
        g = gpu[f].cpu().numpy()
        assert g.shape == h.shape, f
        assert np.array_equal(g.view(np.uint32) if g.dtype == np.float32 else g,
                              h.view(np.uint32) if h.dtype == np.float32 else h), f
    return host


def test_index_dev_baseline_routing(dev):
    """BASELINE configs 4/5 routing: 4096 tokens, top-8 of 256 (Zipf 1.1),
    rank 0 of 8 owns experts 0-31."""
    _say("moe index dev baseline")
    cfg = wl.MoeCfg()
    ids, gates = wl.zipf_routing(cfg.tokens, cfg.experts, cfg.topk, cfg.zipf_s, 6)  # moe_inputs' routing (seed 0)
    host = _check(dev, ids, gates, cfg.e0, cfg.n_local)
    assert host["R"] == 3528 and host["R_pad"] == 6016


@pytest.mark.parametrize("rank", [0, 1, 7])
def test_index_dev_small(dev, rank):
    _say(f"moe index dev small rank={rank}")
    cfg = wl.MoeCfg(tokens=512, H=512, I=256, experts=64, topk=8, ep=8, rank=rank)
    ids, gates = wl.zipf_routing(cfg.tokens, cfg.experts, cfg.topk, cfg.zipf_s, 6)
    _check(dev, ids, gates, cfg.e0, cfg.n_local)


def test_index_dev_edge_cases(dev):
    _say("moe index dev edge cases")
    rng = np.random.default_rng(5)
    # no routed entries at all
    ids = np.full((37, 4), 99, np.int32)
    host = _check(dev, ids, rng.random((37, 4)), 0, 8)
    assert host["R"] == 0 and host["R_pad"] == 0
    # one token; duplicates of a local expert inside a token; all to one expert
    _check(dev, np.array([[3, 1, 3, 7]]), rng.random((1, 4)), 0, 8)
    _check(dev, np.array([[2, 2, 5, 2], [2, 0, 2, 9]]), rng.random((2, 4)), 0, 8)
    _check(dev, np.full((300, 2), 6), rng.random((300, 2)), 0, 8)
    # entry count not a multiple of the 256-entry chunk; experts offset; row_block 64
    ids = rng.integers(0, 40, size=(1001, 3))
    _check(dev, ids, rng.random((1001, 3)), 8, 16)
    _check(dev, ids, rng.random((1001, 3)), 8, 16, row_block=64)
    # more local experts than a plan block's threads
    ids = rng.integers(0, 3000, size=(777, 9))
    _check(dev, ids, rng.random((777, 9)), 100, 1500)


def test_index_dev_feeds_ffn(dev):
    """The device tables drive the fused FFN + combine exactly like the host
    tables (same bytes in, same bytes out)."""
    _say("moe index dev -> ffn")
    cfg = wl.MoeCfg(tokens=256, H=512, I=256, experts=64, topk=8, ep=8, rank=0)
    tokens, ids, gates, w1, w2 = wl.moe_inputs(cfg)
    g = ops.moe_build_indices_dev(torch.from_numpy(np.ascontiguousarray(ids, np.int32)).to(dev),
                                  torch.from_numpy(np.ascontiguousarray(gates, np.float32)).to(dev),
                                  cfg.e0, cfg.n_local)
    h = ops.moe_build_indices(ids, gates, cfg.e0, cfg.n_local)
    hd = {k: torch.from_numpy(np.ascontiguousarray(v)).to(dev) for k, v in h.items() if isinstance(v, np.ndarray)}
    outs = []
    for d in (g, hd):
        Rp = g["R_pad"]
        post = torch.empty((Rp, cfg.H), dtype=torch.bfloat16, device=dev)
        act = torch.empty((Rp, cfg.I), dtype=torch.bfloat16, device=dev)
        ye = torch.empty((Rp, cfg.H), dtype=torch.bfloat16, device=dev)
        y = torch.empty((cfg.tokens, cfg.H), dtype=torch.float32, device=dev)
        ops.moe_ffn_combine(tokens.to(dev), d["pull_indices"], d["row_weight"], d["owner_offset"], d["slot_to_row"],
                            w1.to(dev), w2.to(dev), post, act, ye, y, rb_expert=d["rb_expert"], rb_rows=d["rb_rows"])
        outs.append(y.cpu())
    assert torch.equal(outs[0], outs[1])


# --- the routed layer with the row count left on the device -----------------

LAYER = wl.MoeCfg(tokens=512, H=512, I=256, experts=64, topk=8, ep=8, rank=0)
# GEMM2 with 9 column tiles of 512 (more than 8: the expert tile order)
LAYER_WIDE = wl.MoeCfg(tokens=512, H=4608, I=256, experts=64, topk=8, ep=8, rank=0)


def _host_layer(dev, cfg, tokens, w1, w2, ids, gates, split_ws, fuse):
    """Reference run: host-built tables, host R_pad."""
    h = ops.moe_build_indices(ids, gates, cfg.e0, cfg.n_local)
    d = {k: torch.from_numpy(np.ascontiguousarray(v)).to(dev) for k, v in h.items() if isinstance(v, np.ndarray)}
    Rp = h["R_pad"]
    post = torch.empty((Rp, cfg.H), dtype=torch.bfloat16, device=dev)
    act = torch.empty((Rp, cfg.I), dtype=torch.bfloat16, device=dev)
    ye = torch.empty((Rp, cfg.H), dtype=torch.bfloat16, device=dev)
    y = torch.empty((cfg.tokens, cfg.H), dtype=torch.bfloat16, device=dev)
    ops.moe_ffn_combine(tokens, d["pull_indices"], d["row_weight"], d["owner_offset"], d["slot_to_row"], w1, w2, post,
                        act, ye, y, rb_expert=d["rb_expert"], rb_rows=d["rb_rows"], split_ws=split_ws,
                        fuse_dispatch=fuse)
    return y


class _DeviceLayer:
    """Index build + FFN + combine with every buffer at the row capacity and
    the row count only on the device (nothing read back)."""

    def __init__(self, dev, cfg, tokens, w1, w2, ids_d, gates_d, split_ws, fuse):
        self.cfg, self.tokens, self.w1, self.w2, self.ids, self.gates = cfg, tokens, w1, w2, ids_d, gates_d
        self.split_ws, self.fuse = split_ws, fuse
        T, k = ids_d.shape
        cap = (T * k + cfg.n_local * 127 + 127) // 128 * 128
        self.post = torch.empty((cap, cfg.H), dtype=torch.bfloat16, device=dev)
        self.act = torch.empty((cap, cfg.I), dtype=torch.bfloat16, device=dev)
        self.ye = torch.empty((cap, cfg.H), dtype=torch.bfloat16, device=dev)
        self.y = torch.empty((cfg.tokens, cfg.H), dtype=torch.bfloat16, device=dev)

    def __call__(self):
        c = self.cfg
        t = ops.moe_build_indices_dev(self.ids, self.gates, c.e0, c.n_local, sync=False)
        assert t["pull_indices"].shape[0] == self.post.shape[0]
        ops.moe_ffn_combine(self.tokens, t["pull_indices"], t["row_weight"], t["owner_offset"], t["slot_to_row"],
                            self.w1, self.w2, self.post, self.act, self.ye, self.y, rb_expert=t["rb_expert"],
                            rb_rows=t["rb_rows"], split_ws=self.split_ws, fuse_dispatch=self.fuse, sizes=t["sizes"])
        return self.y


def _routing(cfg, seed):
    ids, gates = wl.zipf_routing(cfg.tokens, cfg.experts, cfg.topk, cfg.zipf_s, seed)
    return np.ascontiguousarray(ids, np.int32), np.ascontiguousarray(gates, np.float32)


@pytest.mark.parametrize("wide", [False, True])
@pytest.mark.parametrize("fuse", [False, True])
def test_layer_with_device_row_count(dev, fuse, wide):
    """Without the K-split every output tile is one workgroup's full-K sum,
    so the capacity-sized launch gives the host-sized launch's bits; with the
    split (planned on the device) it stays within the parity bound.  wide:
    GEMM2 has more than 8 column tiles, so both launches walk the tiles in
    expert order, the device one over its clamped row tiles."""
    _say(f"moe layer, device row count, fuse={fuse} wide={wide}")
    from oracle.gemm import rel_fro
    cfg = LAYER_WIDE if wide else LAYER
    tokens, _, _, w1, w2 = wl.moe_inputs(cfg)
    tokens, w1, w2 = tokens.to(dev), w1.to(dev), w2.to(dev)
    ids, gates = _routing(cfg, 6)
    ids_d, gates_d = torch.from_numpy(ids).to(dev), torch.from_numpy(gates).to(dev)
    ref = _host_layer(dev, cfg, tokens, w1, w2, ids, gates, False, fuse).cpu()
    y = _DeviceLayer(dev, cfg, tokens, w1, w2, ids_d, gates_d, False, fuse)().cpu()
    assert torch.equal(y, ref)
    y_split = _DeviceLayer(dev, cfg, tokens, w1, w2, ids_d, gates_d, None, fuse)().cpu()
    assert rel_fro(y_split.float(), ref.float()) < 1e-2
    # no routed rows at all: R_pad = 0 on the device, every output row zero
    none_d = torch.full_like(ids_d, cfg.experts - 1)
    y0 = _DeviceLayer(dev, cfg, tokens, w1, w2, none_d, gates_d, None, fuse)().cpu()
    assert (y0 == 0).all()


@pytest.mark.parametrize("split", [False, None])
def test_layer_graph_replays(dev, split):
    """The whole routed layer recorded once in a HIP graph and replayed with
    new routings written into the captured inputs; every replay matches an
    eager run on the same routing (bit-exact), with eager library work and
    synchronizations between the replays."""
    _say(f"moe layer graph replays split={split}")
    cfg = LAYER
    tokens, _, _, w1, w2 = wl.moe_inputs(cfg)
    tokens, w1, w2 = tokens.to(dev), w1.to(dev), w2.to(dev)
    ids0, gates0 = _routing(cfg, 6)
    ids_d, gates_d = torch.from_numpy(ids0).to(dev), torch.from_numpy(gates0).to(dev)
    layer = _DeviceLayer(dev, cfg, tokens, w1, w2, ids_d, gates_d, split, False)
    eager = {}
    for seed in (6, 7, 8):
        ids, gates = _routing(cfg, seed)
        ids_d.copy_(torch.from_numpy(ids)); gates_d.copy_(torch.from_numpy(gates))
        eager[seed] = layer().clone()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        layer()
    for seed in (7, 6, 8, 7):
        ids, gates = _routing(cfg, seed)
        ids_d.copy_(torch.from_numpy(ids)); gates_d.copy_(torch.from_numpy(gates))
        layer.y.fill_(-1.0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(layer.y, eager[seed]), seed
        # eager library work between replays
        ops.gemm(tokens[:256], w1[0, :, :256].contiguous())
        torch.cuda.synchronize()


def test_index_dev_random_routings(dev):
    """Seeded random routings: token count, top-k, expert count, local
    expert window and row block; every table bit-identical to the host
    builder."""
    rng = np.random.default_rng(4321)
    for case in range(12):
        T = int(rng.integers(1, 9000))
        topk = int(rng.integers(1, 10))
        experts = int(rng.choice([8, 64, 256, 1024]))
        n_local = int(rng.integers(1, experts + 1))
        e0 = int(rng.integers(0, experts - n_local + 1))
        row_block = int(rng.choice([64, 128]))
        _say(f"moe index dev random case={case} T={T} topk={topk} E={experts} e0={e0} n_local={n_local} rb={row_block}")
        ids, gates = wl.zipf_routing(T, experts, min(topk, experts), float(rng.choice([0.0, 1.1])), 700 + case)
        _check(dev, ids, gates, e0, n_local, row_block)
