"""CPU oracle — TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference's Core chains for the fused per-layer kernels, used
as the checker for the HIP kernels. Only `tests/`, `__graft_entry__.smoke()` and
`bench.py`'s `cpu_baseline` leg may import it; the product path (`mlx-omnia_amd/`) never
does, and fails loudly instead of falling back here when its HIP library is missing.

Each function cites the reference file:line whose arithmetic it restates. Every function
is pinned by tests under `tests/test_oracle_*.py` against checks independent of its own
formula: library routines (torch's bf16 conversion, rms_norm, complex rotation, silu,
softplus, stable sort, embedding), invariants (identity rotation at position 0, norm
preservation, verbatim tails, ordering), closed forms in fp64, and the reference's own
known-answer tie fixtures.

bf16 values travel as uint16 bit patterns, fp32 as float32, exactly as through the C ABI.
"""
