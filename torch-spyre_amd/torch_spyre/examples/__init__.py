"""Workloads that exercise the spyre device end to end (the decoder configs
the benchmark and the tests run)."""
