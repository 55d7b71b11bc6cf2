"""CPU oracle for the pjrtx hot path — TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference's semantics for each hot-path op, used
by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
checker. The product path (pjrtx_amd, libpjrtx_rocm_plugin.so) never imports
or calls anything here, and has no CPU fallback.
"""
