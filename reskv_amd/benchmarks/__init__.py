"""Benchmark commands: ``kernels`` (API sweep), ``inference`` (one local
checkpoint, ResKV or dense), ``compare`` (sequential runs and report
validation); ``timing`` (the timed greedy decode) and ``common`` are shared."""
