"""Measurement programs that build instrumented copies of the library's kernels."""
