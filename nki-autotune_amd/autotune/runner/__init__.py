"""Profiling backend (hipEvent timing) of the autotune loop."""
