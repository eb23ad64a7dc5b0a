"""Autotune for the MI355X kernel_library: sweep tile configs, profile, select the fastest.

Public surface (reference autotune/src/autotune/__init__.py and
autotune/src/autotune/runner/):

* ``autotune.runner.api.profile`` -- build + time ``KernelJob`` s on the GPU,
  return a ``ProfileOutput`` (results table, ``successes``, ``failures``,
  ``best``) and write the cache layout with ``results.json``.
* ``autotune.tune.tune`` -- the sweep-and-select loop over the tile grid.
"""
