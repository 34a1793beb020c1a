"""CPU oracle for the pagoda decode path (TEST INFRASTRUCTURE ONLY).

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
never by the product package pagoda_amd/.
"""
