"""Measurement and correctness helpers shared by tests and benchmarks."""
