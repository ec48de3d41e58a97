"""CPU oracle for the decode-step hot path — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, what strata-mlx computes on the path the HIP library replaces: the
dequantization of the ten GGUF block types, the expert products, the router's top-k and weights, SwiGLU,
the MoE block's combine, the prompt tiles and paged decode attention. Every function cites the reference
file:line it follows (paths relative to the strata-mlx repository).

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import it, and only
to check results or as the reported CPU baseline — never as the thing measured or shipped. The product package
(`strata_hip`) does not import it and fails loudly when its HIP library is missing.

Parity status of each function is stated in its docstring; "parity unpinned" marks content that no
golden vector, reference test or closed form in this container can check (the ggml codebook grids, which
strata-mlx reads from gguf-py 0.19.0 at run time and which is not installed here).
"""
