"""CPU oracle of the tallax sort / select / sample path (test infrastructure only).

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, always as the checker; the product package never imports it.
"""
