"""Seeded synthetic inputs for the BASELINE configurations.

Shapes and distributions are the ones BASELINE.json defines; all draws come
from seeded generators so the HIP path and the CPU oracle see identical
tensors.  Routing is Zipf(s) expert popularity with Gumbel-top-k selection
(sampling k distinct experts with probability proportional to popularity —
the same without-replacement draw as the reference's
``torch.multinomial(..., replacement=False)``, reference
bench/dispatch_gemm_bench.py:103-124) and softmax gates over the k chosen
logits.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

ROW_BLOCK = 128


def randn_bf16(shape, seed: int, scale: float = 1.0, device="cpu") -> torch.Tensor:
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
    if scale != 1.0:
        x.mul_(scale)
    return x.to(torch.bfloat16)


def stage_order(n: int, seed: int) -> np.ndarray:
    """Seeded permutation of n tiles: the order the producer publishes them."""
    return np.random.default_rng(seed).permutation(n).astype(np.int32)


def zipf_routing(num_tokens: int, num_experts: int, topk: int, s: float = 1.1, seed: int = 6):
    """Returns (topk_ids int32 [T, k], gates float32 [T, k])."""
    rng = np.random.default_rng(seed)
    ranks = rng.permutation(num_experts) + 1
    logp = -s * np.log(ranks.astype(np.float64))
    logits = logp[None, :] + rng.gumbel(size=(num_tokens, num_experts))
    ids = np.argsort(-logits, axis=1, kind="stable")[:, :topk]
    sel = np.take_along_axis(logits, ids, 1)
    sel = sel - sel.max(axis=1, keepdims=True)
    w = np.exp(sel)
    gates = (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
    return ids.astype(np.int32), gates


@dataclass(frozen=True)
class GemmCfg:
    M: int = 4096
    N: int = 4096
    K: int = 4096


@dataclass(frozen=True)
class AgCfg:
    world: int = 8
    shard_rows: int = 2048
    K: int = 8192
    N: int = 3584

    @property
    def M(self) -> int:
        return self.world * self.shard_rows


@dataclass(frozen=True)
class RsCfg:
    world: int = 8
    rank: int = 0
    M: int = 16384
    K: int = 3584
    N: int = 8192
    peer_std: float = 0.5


@dataclass(frozen=True)
class MoeCfg:
    tokens: int = 4096
    H: int = 7168
    I: int = 2048
    experts: int = 256
    topk: int = 8
    ep: int = 8
    rank: int = 0
    zipf_s: float = 1.1

    @property
    def n_local(self) -> int:
        return self.experts // self.ep

    @property
    def e0(self) -> int:
        return self.rank * self.n_local


def gemm_inputs(cfg: GemmCfg, device="cpu", seed=0):
    A = randn_bf16((cfg.M, cfg.K), seed, cfg.K ** -0.5, device)
    B = randn_bf16((cfg.K, cfg.N), seed + 1, cfg.K ** -0.5, device)
    return A, B


def ag_inputs(cfg: AgCfg, device="cpu", seed=0):
    """A_shards [M, K] (the world row shards stacked in rank order), B [K, N],
    stage order over the M/128 row tiles (seed+2)."""
    A = randn_bf16((cfg.M, cfg.K), seed, cfg.K ** -0.5, device)
    B = randn_bf16((cfg.K, cfg.N), seed + 1, cfg.K ** -0.5, device)
    order = stage_order(cfg.M // ROW_BLOCK, seed + 2)
    return A, B, order


def rs_inputs(cfg: RsCfg, device="cpu", seed=0):
    """A [M, K], B [K, N], peer partials [world-1, M/world, N] ~ N(0, std),
    stage order over the (world-1) * (M/world)/128 peer tiles."""
    A = randn_bf16((cfg.M, cfg.K), seed, cfg.K ** -0.5, device)
    B = randn_bf16((cfg.K, cfg.N), seed + 1, cfg.K ** -0.5, device)
    rows = cfg.M // cfg.world
    peers = randn_bf16((cfg.world - 1, rows, cfg.N), seed + 3, cfg.peer_std, device)
    order = stage_order((cfg.world - 1) * rows // ROW_BLOCK, seed + 4)
    return A, B, peers, order


def moe_inputs(cfg: MoeCfg, device="cpu", seed=0, with_w2: bool = True):
    """tokens [T, H] ~ N(0,1); routing (ids, gates); w1 [E_loc, H, 2I] and
    w2 [E_loc, I, H] ~ N(0, 1/sqrt(K))."""
    tokens = randn_bf16((cfg.tokens, cfg.H), seed + 5, 1.0, device)
    ids, gates = zipf_routing(cfg.tokens, cfg.experts, cfg.topk, cfg.zipf_s, seed + 6)
    w1 = randn_bf16((cfg.n_local, cfg.H, 2 * cfg.I), seed + 7, cfg.H ** -0.5, device)
    w2 = randn_bf16((cfg.n_local, cfg.I, cfg.H), seed + 8, cfg.I ** -0.5, device) if with_w2 else None
    return tokens, ids, gates, w1, w2
