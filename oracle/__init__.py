"""CPU oracle for the transformer-layer-stack forward.

TEST INFRASTRUCTURE ONLY. Nothing in the product (`techjam2026_amd/`) imports
this package. Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline`
leg of `bench.py` may use it, and only as the checker, never as the thing that
is measured or shipped.

Modules:

* `reference` -- a functional restatement of the organizer's reference layer
  (`torch_transformer_benchmark.py:59-172`) over a plain state dict, in fp32 or
  fp64, with a naive attention and a query-chunked O(S) attention
  (`scripts/shape14.py:124-166`, extended with the key-padding mask and the
  three row masks the reference applies).
* `brute` -- pure-Python loops (math.erf / math.exp / math.sqrt in Python
  floats) for tiny shapes. It shares no code with `reference` and pins it.

Parity pinning (how each oracle function is checked before it is trusted) is
listed in `tests/test_oracle.py`: closed forms (LN(0) = beta, S=1 identity,
masked rows zero), textbook library routines (`F.layer_norm`, `F.gelu`,
`F.scaled_dot_product_attention`), brute force on tiny inputs, and
chunked == naive on ragged chunk sizes.
"""
