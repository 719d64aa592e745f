"""Float32 CPU restatement of the GEMM-shaped parts of the path (test-only).

Each function follows the torch reference the reference's own bench uses:
* gemm_ref          — ``C_ref = A_gathered @ B`` (reference bench/ag_gemm_bench.py:386-400)
* ag_gemm_ref       — the same on the shards gathered in rank order
* gemm_rs_ref       — per-rank partial, then the sum over ranks of the owned
                      slice (reference bench/gemm_rs_bench.py:820-867); here the
                      peers' partials are given inputs, summed in fp32.
Inputs are bf16 tensors (values exactly representable); the oracle widens them
to float32 and multiplies in float32, as BASELINE's "float32 CPU torch
reference on identical seeded inputs" requires.
"""
from __future__ import annotations

import torch


def gemm_ref(A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    """C = A @ B in float32 on the CPU."""
    return A.detach().cpu().float() @ B.detach().cpu().float()


def gemm_bruteforce(A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    """Triple loop in Python floats (double precision) — tiny shapes only."""
    a = A.cpu().float().tolist()
    b = B.cpu().float().tolist()
    M, K, N = len(a), len(b), len(b[0])
    out = [[sum(a[i][k] * b[k][j] for k in range(K)) for j in range(N)] for i in range(M)]
    return torch.tensor(out, dtype=torch.float64)


def ag_gemm_ref(shards: list[torch.Tensor] | torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    """AllGather then GEMM: concatenate the row shards in rank order."""
    A = torch.cat([s.cpu() for s in shards], 0) if isinstance(shards, (list, tuple)) else shards
    return gemm_ref(A, B)


def gemm_rs_ref(A: torch.Tensor, B: torch.Tensor, peer_partials: torch.Tensor, rank: int, world: int):
    """Returns (partial fp32 [M,N], owned fp32 [M/world,N]).

    owned = partial[rank rows] + sum_p peer_partials[p]  (fp32, p ascending)."""
    P = gemm_ref(A, B)
    rows = P.shape[0] // world
    owned = P[rank * rows:(rank + 1) * rows].clone()
    for p in range(peer_partials.shape[0]):
        owned += peer_partials[p].cpu().float()
    return P, owned


def gemm_ar_ref(A: torch.Tensor, B: torch.Tensor, peer_partials: torch.Tensor) -> torch.Tensor:
    """All-reduce at one rank's share: A@B (fp32) + sum_p peer_partials[p]
    (fp32, p ascending) over every row — the reference checks its C_final
    against all_reduce(SUM) of the ranks' matmuls
    (bench/gemm_ar_bench.py:510-514)."""
    out = gemm_ref(A, B)
    for p in range(peer_partials.shape[0]):
        out += peer_partials[p].cpu().float()
    return out


def rel_fro(x: torch.Tensor, ref: torch.Tensor) -> float:
    """Relative Frobenius error ||x - ref||_F / ||ref||_F (float64)."""
    x = x.detach().cpu().double()
    ref = ref.detach().cpu().double()
    den = torch.linalg.norm(ref)
    num = torch.linalg.norm(x - ref)
    return float(num / den) if den > 0 else float(num)
