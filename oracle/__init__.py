"""CPU oracle for libmk — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import anything under ``oracle/``; the product (``mkernel_amd``) never
does and fails loudly when its HIP library is missing.

Contents
--------
* :mod:`oracle.gemm` — float32 CPU torch restatement of the GEMM core, the
  AllGather+GEMM result and the GEMM+ReduceScatter fold.
* :mod:`oracle.moe`  — routing-index build (pure Python and numpy), permute,
  SwiGLU FFN and gather-combine.
* ``oracle/moe_index.c`` — an independent plain-C restatement of the index
  build (built by ``oracle/Makefile`` into ``oracle/_build/``), used to
  cross-check the Python restatement and libmk's C++ builder bit-exactly.

How each function is pinned (there are no golden vectors in the reference —
it has no tests directory; its checks are the torch references inside
``bench/*.py``):

* gemm_ref: brute-force triple loop on tiny shapes, identity/zero-row special
  cases, transpose identity (tests/test_oracle.py).
* ag_gemm_ref: equals gemm_ref on the gathered A; independent of stage order.
* gemm_rs_ref: known answer "all partials equal => world x partial"; sum order.
* routing indices: hand-worked tiny example (tests/golden/index_tiny.json),
  pure-Python vs numpy vs C restatement, and invariants (every local (t,k)
  exactly once, padding rows -1, padded counts multiples of 128, CSR sums).
* silu_mul: odd-part identity silu(x) - silu(-x) = x, silu(0) = 0, limits.
* combine_ref: one-hot routing reduces to a row copy scaled by the gate;
  linearity in the weights.
"""
