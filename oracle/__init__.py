"""CPU oracle of the spiking decode hot path -- TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, as the checker (never as the thing measured on the GPU, never shipped).
"""
