"""CPU oracle for the Wafer Reference backend semantics.

Test infrastructure only: tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use it as the checker or as the timed CPU lane.  The HIP
product path in vibe_compiler_amd/ never imports it.
"""
