"""CPU oracle of the reference DIA algorithms -- TEST INFRASTRUCTURE ONLY.

May be imported only by tests/, __graft_entry__.smoke() and the cpu_baseline
leg of bench.py, and only as the checker / the CPU baseline, never as the
thing measured or shipped.
"""
