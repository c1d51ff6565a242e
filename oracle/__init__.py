"""CPU oracle for the vortx linalg hot path — TEST INFRASTRUCTURE ONLY.

Imported only by tests/, ``__graft_entry__.smoke()`` and bench.py's
cpu_baseline leg. The product package ``vortx_amd`` never imports it.
"""
