"""Seeded random cases on the GPU (bounded count, small sizes): GEMM shapes,
grid caps and tile heights against the oracle; random MoE routings through
the device index build and the fused FFN + combine against the oracle."""
import numpy as np
import pytest
import torch

from mkernel_amd import ops, workloads as wl
from oracle import moe as om
from oracle.gemm import gemm_ref, rel_fro

pytestmark = pytest.mark.gpu
TOL = 2e-2


@pytest.mark.parametrize("seed", range(12))
def test_random_gemm_shapes(dev, seed):
    rng = np.random.default_rng(100 + seed)
    tile = int(rng.choice([0, 128, 256]))
    mb = 256 if tile == 256 else 128
    M = mb * int(rng.integers(1, 9))
    N = 256 * int(rng.integers(1, 6))
    K = 32 * int(rng.integers(1, 40))
    cus = int(rng.choice([0, 0, 7, 64, 130]))
    print(f"random gemm seed={seed} M={M} N={N} K={K} tile={tile} cus={cus}", flush=True)
    A = wl.randn_bf16((M, K), 200 + seed, K ** -0.5)
    B = wl.randn_bf16((K, N), 300 + seed, K ** -0.5)
    C = ops.gemm(A.to(dev), B.to(dev), tile_m=tile, num_cus=cus)
    torch.cuda.synchronize()
    ref = gemm_ref(A, B)
    assert rel_fro(C.float(), ref) < TOL
    assert torch.allclose(C.cpu().float(), ref, rtol=2 ** -7, atol=1e-5)


@pytest.mark.parametrize("seed", range(6))
def test_random_moe_layer(dev, seed):
    rng = np.random.default_rng(400 + seed)
    T = int(rng.integers(1, 300))
    E = int(rng.choice([16, 32, 64]))
    ep = int(rng.choice([2, 4, 8]))
    k = int(rng.integers(1, 9))
    H = 256 * int(rng.integers(1, 3))
    I = 128 * int(rng.integers(1, 3))
    rank = int(rng.integers(0, ep))
    n_local = E // ep
    print(f"random moe seed={seed} T={T} E={E} ep={ep} k={k} H={H} I={I} rank={rank}", flush=True)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    gates = rng.random((T, k), dtype=np.float32)
    tokens = wl.randn_bf16((T, H), 500 + seed)
    w1 = wl.randn_bf16((n_local, H, 2 * I), 600 + seed, H ** -0.5)
    w2 = wl.randn_bf16((n_local, I, H), 700 + seed, I ** -0.5)
    d = ops.moe_build_indices_dev(torch.from_numpy(ids).to(dev), torch.from_numpy(gates).to(dev), rank * n_local,
                                  n_local)
    Rp = d["R_pad"]
    host = ops.moe_build_indices(ids, gates, rank * n_local, n_local)
    assert Rp == host["R_pad"] and d["R"] == host["R"]
    y = torch.empty((T, H), dtype=torch.float32, device=dev)
    if Rp == 0:
        return
    act = torch.empty((Rp, I), dtype=torch.bfloat16, device=dev)
    ye = torch.empty((Rp, H), dtype=torch.bfloat16, device=dev)
    ops.moe_ffn_combine(tokens.to(dev), d["pull_indices"], d["row_weight"], d["owner_offset"], d["slot_to_row"],
                        w1.to(dev), w2.to(dev), None, act, ye, y, rb_expert=d["rb_expert"], rb_rows=d["rb_rows"],
                        fuse_dispatch=True)
    torch.cuda.synchronize()
    post = om.permute_ref(tokens, host["pull_indices"])
    _, ye_ref = om.ffn_ref(post, w1, w2, host["padded_tokens_per_expert"], I)
    y_ref = om.combine_ref(ye_ref, host["row_weight"], host["pull_indices"], T)
    if float(y_ref.abs().max()) == 0.0:
        assert float(y.abs().max()) == 0.0
    else:
        assert rel_fro(y, y_ref) < TOL
