"""TEST INFRASTRUCTURE ONLY: the CPU oracle for the KV data path. See kv_oracle.c.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this package.
The product package (layover_amd) never does.
"""
