"""CPU oracle for the hot path -- TEST INFRASTRUCTURE ONLY.

Used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg;
never by the product package barracuda_amd/.
"""
