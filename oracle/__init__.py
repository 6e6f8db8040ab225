"""CPU oracle for the ``awq_inference_engine`` hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``qvggt_amd``) may import
this package.  It is imported by ``tests/``, by ``__graft_entry__.smoke()``
and by the ``cpu_baseline`` leg of ``bench.py`` -- always as the checker or
the reported CPU baseline, never as the thing measured or shipped.

Each module restates one part of the reference algorithm in plain numpy and
cites the reference file:line it follows (paths relative to the reference
repository root, ``qvggt/runtime/...``).  How each function is pinned is
listed in the module docstrings; a function with no independent check says
"parity unpinned".
"""
