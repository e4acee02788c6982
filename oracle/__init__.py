"""CPU parity oracle for the quantized decode path — TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() (as the checker) and the
cpu_baseline leg of bench.py.  The product package llm_core_amd never imports
it.  See oracle/axf_oracle.h for what it restates and how it is pinned.
"""
