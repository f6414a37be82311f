"""Checker-side CPU restatements of the reference (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker or the CPU baseline -- never as
the product path.  See af2.py (the JAX trunk) and jax_prng.py (jax.random).
"""
