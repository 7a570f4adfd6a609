"""Benchmark harness (counterpart of the reference's ``benchmarks`` package):
``kernels`` (API sweep), ``inference`` (one checkpoint, ResKV or dense),
``compare`` (sequential runs plus report validation) and the shared ``timing``."""
