"""Kernel-level UOp graphs, their lowering to linear listings, and scheduled-matmul rewriting."""
