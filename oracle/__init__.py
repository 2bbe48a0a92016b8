"""CPU oracle for the quantized-GEMM / fused-MoE hot path.

TEST INFRASTRUCTURE ONLY. Nothing in the product (`vllm-torchtpu_amd/qmoe`)
imports this package. Only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may use it, and only as the checker.

Each function restates, in numpy (float32 / float64 / integer arithmetic), the
algorithm of the reference plugin `vllm_torchtpu` at the file:line cited in its
docstring (paths relative to `src/vllm_torchtpu/` of the reference). The
reference itself cannot be imported here (JAX / torch_tpu / vLLM are absent),
so each function is pinned instead by:

* the known-answer vectors of the reference's own tests (cited per test in
  `tests/test_oracle_*.py`),
* closed forms and library routines (torch's float8 casts, `np.argsort`
  stable sort, brute-force loops on tiny inputs), and
* invariants (round trips, monotonicity, permutation properties).

Functions whose result no such check fixes say "parity unpinned" in their
docstring; the list is:

* ``quantize_block_int8`` saturation of a code that rounds to +128 (the
  reference's bf16 quotient can reach 127.5; its XLA float->int8 cast is
  assumed saturating).
* ``grouped_topk`` (upstream vLLM, not vendored in the reference; restated
  from the DeepSeek-V3 method, see its docstring).
"""

from oracle import codecs, linear, moe, quant, routing  # noqa: F401
