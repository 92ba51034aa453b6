"""CPU oracle for the xinfer attention hot path -- TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference operators' arithmetic, used by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker.  The
product path (xinfer_amd) never imports it.  See oracle/attention.py.
"""
