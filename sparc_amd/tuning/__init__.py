"""GEMM solution choices for the block stack's projections (TunableOp results
files measured on MI355X)."""
