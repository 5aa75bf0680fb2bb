"""CPU oracle of the jointkv hot path — test infrastructure only.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, as the checker or the timed CPU baseline; never by the product package.
"""
