"""Profiling backend of the autotune loop: hipcc / prebuilt instances, hipEvent timing, results.json."""
