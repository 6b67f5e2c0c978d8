"""CPU oracle (test infrastructure only): a C++ restatement of Camelid's CPU forward.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use it.
"""
