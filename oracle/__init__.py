"""CPU oracle for the paged-attention and gated-delta hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports, links or
executes this package.  It may be used only by ``tests/``, by
``__graft_entry__.smoke()`` and by the ``cpu_baseline`` leg of ``bench.py``, and
there only as the checker (or as the timed CPU baseline), never as the thing
that is measured or shipped.

Every function restates an algorithm of the reference runtime
(``lvyufeng/Qwen3.6-2080ti``) in this repository's own code and cites the
reference ``file:line`` it follows.  Integer and byte work (slot indexing, block
tables, gathers) is bit-exact NumPy / plain Python; floating-point work uses
PyTorch CPU kernels with the reference's dtype cast points, because PyTorch CPU
is the arithmetic the reference itself runs on.

Pinning status (what checks each function against something other than its own
formula) is recorded per function in the module docstrings and enforced by
``tests/test_oracle_*.py``.
"""
