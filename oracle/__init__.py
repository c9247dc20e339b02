"""CPU oracle of molten's quantized-matmul path: TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, as the checker; the product (molten_amd/) never imports it.
"""
